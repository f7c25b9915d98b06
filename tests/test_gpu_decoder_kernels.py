"""The decode-step kernels of the greedy-decode harness (csrc/qs_decoder.hip)
against the transformers / torch ops they replace: Qwen3RMSNorm with the
residual add, q/k norm + rotary embedding + cache write, attention over the
filled cache prefix (reference in fp32 on the CPU), and act_fn(gate) * up;
and the same norm done inside a grouped one-launch forward
(qs_linear_forward_group_pre), bit-identical to the separate launches."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from quipsharp_amd import _lib
    return _lib, _lib.lib()


def _bf16_ulps(a, b):
    """Largest distance in bf16 units in the last place between two bf16 tensors."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    # order-preserving map of the sign-magnitude bit patterns
    ia = torch.where(ia < 0, -32768 - ia, ia)
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return int((ia - ib).abs().max().item())


@pytest.mark.parametrize("rows,dim", [(1, 5120), (8, 5120), (3, 512), (2, 520), (1, 20480), (2, 32768)])
def test_rmsnorm_with_residual(dev, rows, dim):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    lib, L = _lib()
    g = torch.Generator().manual_seed(rows)
    h = (torch.randn(rows, dim, generator=g) * 3).bfloat16().to(dev)
    d = torch.randn(rows, dim, generator=g).bfloat16().to(dev)
    norm = Qwen3RMSNorm(dim, eps=1e-6).to(dev).bfloat16()
    with torch.no_grad():
        norm.weight.copy_((1 + 0.1 * torch.randn(dim, generator=g)).bfloat16())
        want_h = h + d
        want_x = norm(want_h)
    hh = h.clone()
    x = torch.empty_like(h)
    lib.check(L.qs_dec_rmsnorm(lib.ptr(hh), lib.ptr(d), lib.ptr(hh), lib.ptr(norm.weight), lib.ptr(x), rows, dim, dim,
                               1e-6, lib.stream_of(h)))
    torch.cuda.synchronize()
    assert torch.equal(hh, want_h)
    assert _bf16_ulps(x, want_x) <= 1
    # no residual: h untouched
    x2 = torch.empty_like(h)
    lib.check(L.qs_dec_rmsnorm(lib.ptr(h), None, None, lib.ptr(norm.weight), lib.ptr(x2), rows, dim, dim, 1e-6,
                               lib.stream_of(h)))
    torch.cuda.synchronize()
    with torch.no_grad():
        assert _bf16_ulps(x2, norm(h)) <= 1


@pytest.mark.parametrize("rows,nh,nkv", [(1, 64, 8), (8, 64, 8), (2, 4, 2)])
def test_qk_norm_rope_cache(dev, rows, nh, nkv):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb
    lib, L = _lib()
    max_len, p = 96, 37
    cfg = Qwen3Config(hidden_size=nh * 128, num_attention_heads=nh, num_key_value_heads=nkv, head_dim=128)
    rot = Qwen3RotaryEmbedding(cfg).to(dev)
    g = torch.Generator().manual_seed(nh + rows)
    q = torch.randn(rows, nh * 128, generator=g).bfloat16().to(dev)
    k = torch.randn(rows, nkv * 128, generator=g).bfloat16().to(dev)
    v = torch.randn(rows, nkv * 128, generator=g).bfloat16().to(dev)
    qn, kn = Qwen3RMSNorm(128).to(dev).bfloat16(), Qwen3RMSNorm(128).to(dev).bfloat16()
    with torch.no_grad():
        qn.weight.copy_((1 + 0.1 * torch.randn(128, generator=g)).bfloat16())
        kn.weight.copy_((1 + 0.1 * torch.randn(128, generator=g)).bfloat16())
        cos, sin = rot(torch.zeros(1, 1, 8, device=dev, dtype=torch.bfloat16), torch.arange(max_len, device=dev)[None])
        cos_t, sin_t = cos[0].contiguous(), sin[0].contiguous()
        qs = qn(q.view(rows, 1, nh, 128)).transpose(1, 2)
        ks = kn(k.view(rows, 1, nkv, 128)).transpose(1, 2)
        qr, kr = apply_rotary_pos_emb(qs, ks, cos[:, p:p + 1], sin[:, p:p + 1])
    kc = torch.zeros(rows, nkv, max_len, 128, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty(rows, nh * 128, dtype=torch.bfloat16, device=dev)
    pos = torch.full((1,), p, dtype=torch.long, device=dev)
    lib.check(L.qs_dec_qk_norm_rope(lib.ptr(q), lib.ptr(k), lib.ptr(v), lib.ptr(qn.weight), lib.ptr(kn.weight),
                                    lib.ptr(cos_t), lib.ptr(sin_t), lib.ptr(pos), lib.ptr(qo), lib.ptr(kc), lib.ptr(vc),
                                    rows, nh, nkv, 128, max_len, 1e-6, lib.stream_of(q)))
    torch.cuda.synchronize()
    assert _bf16_ulps(qo.view(rows, nh, 128), qr[:, :, 0]) <= 1
    assert _bf16_ulps(kc[:, :, p], kr[:, :, 0]) <= 1
    assert torch.equal(vc[:, :, p], v.view(rows, nkv, 128))
    # nothing else of the caches is written
    assert kc[:, :, :p].abs().sum().item() == 0 and vc[:, :, p + 1:].abs().sum().item() == 0


@pytest.mark.parametrize("rows,nh,nkv,length,max_len", [(1, 64, 8, 1, 770), (1, 64, 8, 64, 770), (1, 64, 8, 577, 770),
                                                        (8, 64, 8, 300, 770), (2, 4, 2, 130, 770),
                                                        (1, 64, 8, 4100, 4160)])
def test_attention_over_prefix(dev, rows, nh, nkv, length, max_len):
    """Against fp32 attention on the CPU; fills of one position, a whole
    split, partial splits, and 65 splits of a longer cache."""
    lib, L = _lib()
    g = torch.Generator().manual_seed(length)
    q = torch.randn(rows, nh, 128, generator=g).bfloat16()
    kc = torch.randn(rows, nkv, max_len, 128, generator=g).bfloat16()
    vc = torch.randn(rows, nkv, max_len, 128, generator=g).bfloat16()
    # positions past the filled length hold large values that must not leak in
    kc[:, :, length:] = 1e4
    vc[:, :, length:] = 1e4
    scale = 128 ** -0.5
    G = nh // nkv
    kk = kc[:, :, :length].float().repeat_interleave(G, dim=1)
    vv = vc[:, :, :length].float().repeat_interleave(G, dim=1)
    s = torch.einsum("bhd,bhpd->bhp", q.float(), kk) * scale
    want = torch.einsum("bhp,bhpd->bhd", torch.softmax(s, -1), vv).reshape(rows, nh * 128)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    out = torch.empty(rows, nh * 128, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(int(L.qs_dec_attention_workspace_bytes(rows, nkv, max_len)), dtype=torch.uint8, device=dev)
    pos = torch.full((1,), length - 1, dtype=torch.long, device=dev)
    lib.check(L.qs_dec_attention(lib.ptr(qd), lib.ptr(kd), lib.ptr(vd), lib.ptr(pos), lib.ptr(out), nh * 128,
                                 lib.ptr(ws), ws.numel(), rows, nh, nkv, 128, max_len, scale, lib.stream_of(qd)))
    torch.cuda.synchronize()
    got = out.float().cpu()
    rel = ((got - want).norm() / want.norm()).item()
    assert rel < 1e-2, rel
    assert (got - want).abs().max().item() < 0.05


@pytest.mark.parametrize("rows,nh,nkv,pos", [(1, 64, 8, 0), (1, 64, 8, 63), (1, 64, 8, 64), (1, 64, 8, 577),
                                             (8, 64, 8, 300), (2, 4, 2, 130), (3, 40, 8, 769)])
def test_attention_rope_equals_separate(dev, rows, nh, nkv, pos):
    """qs_dec_attention_rope (q/k norm + rotary inside the attention's split
    launch) gives the bits of qs_dec_qk_norm_rope then qs_dec_attention: the
    output, the key and value caches at pos, and nothing else of the caches
    written.  Positions at a split's first and last slot and the cache's end."""
    lib, L = _lib()
    max_len = 770
    g = torch.Generator().manual_seed(pos + rows)
    q = torch.randn(rows, nh * 128, generator=g).bfloat16().to(dev)
    k = torch.randn(rows, nkv * 128, generator=g).bfloat16().to(dev)
    v = torch.randn(rows, nkv * 128, generator=g).bfloat16().to(dev)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16().to(dev)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16().to(dev)
    ang = torch.arange(max_len)[:, None] * (1e6 ** (-torch.arange(64) / 64))[None]
    cos_t = torch.cat([ang.cos(), ang.cos()], 1).bfloat16().to(dev)
    sin_t = torch.cat([ang.sin(), ang.sin()], 1).bfloat16().to(dev)
    kc0 = torch.randn(rows, nkv, max_len, 128, generator=g).bfloat16().to(dev)
    vc0 = torch.randn(rows, nkv, max_len, 128, generator=g).bfloat16().to(dev)
    # rows from pos on are not filled yet: NaN must not reach the output
    # (the new row's stale cache value is replaced by the new key / value,
    # and rows past it only ever meet a zero probability through clamping)
    kc0[:, :, pos:] = float("nan")
    vc0[:, :, pos:] = float("nan")
    p = torch.full((1,), pos, dtype=torch.long, device=dev)
    ws = torch.empty(int(L.qs_dec_attention_workspace_bytes(rows, nkv, max_len)), dtype=torch.uint8, device=dev)
    st = lib.stream_of(q)
    scale = 128 ** -0.5
    kc1, vc1 = kc0.clone(), vc0.clone()
    qn = torch.empty_like(q)
    want = torch.empty_like(q)
    lib.check(L.qs_dec_qk_norm_rope(lib.ptr(q), lib.ptr(k), lib.ptr(v), lib.ptr(qw), lib.ptr(kw), lib.ptr(cos_t),
                                    lib.ptr(sin_t), lib.ptr(p), lib.ptr(qn), lib.ptr(kc1), lib.ptr(vc1), rows, nh, nkv,
                                    128, max_len, 1e-6, st))
    lib.check(L.qs_dec_attention(lib.ptr(qn), lib.ptr(kc1), lib.ptr(vc1), lib.ptr(p), lib.ptr(want), nh * 128,
                                 lib.ptr(ws), ws.numel(), rows, nh, nkv, 128, max_len, scale, st))
    kc2, vc2 = kc0.clone(), vc0.clone()
    got = torch.empty_like(q)
    lib.check(L.qs_dec_attention_rope(lib.ptr(q), lib.ptr(k), lib.ptr(v), lib.ptr(qw), lib.ptr(kw), lib.ptr(cos_t),
                                      lib.ptr(sin_t), lib.ptr(p), lib.ptr(kc2), lib.ptr(vc2), lib.ptr(got), nh * 128,
                                      lib.ptr(ws), ws.numel(), rows, nh, nkv, 128, max_len, 1e-6, scale, st))
    torch.cuda.synchronize()
    assert torch.isfinite(want).all()
    assert torch.equal(got, want)
    bits = lambda t: t.view(torch.int16)  # noqa: E731  (NaN rows compare by their bits)
    assert torch.equal(bits(kc2), bits(kc1)) and torch.equal(bits(vc2), bits(vc1))
    # the separate path wrote the new position and nothing else
    assert torch.equal(vc1[:, :, pos], v.view(rows, nkv, 128))
    keep = torch.ones(max_len, dtype=torch.bool, device=dev)
    keep[pos] = False
    assert torch.equal(bits(kc2[:, :, keep]), bits(kc0[:, :, keep]))
    assert torch.equal(bits(vc2[:, :, keep]), bits(vc0[:, :, keep]))


def test_position_past_the_cache_writes_nothing(dev):
    """pos = max_len: the kernels see it on the device and leave the caches
    and the output untouched."""
    lib, L = _lib()
    rows, nh, nkv, max_len = 1, 8, 2, 128
    g = torch.Generator().manual_seed(5)
    q = torch.randn(rows, nh * 128, generator=g).bfloat16().to(dev)
    kv = torch.randn(rows, nkv * 128, generator=g).bfloat16().to(dev)
    w = torch.ones(128, dtype=torch.bfloat16, device=dev)
    tab = torch.ones(max_len, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.randn(rows, nkv, max_len, 128, generator=g).bfloat16().to(dev)
    vc = kc.clone()
    kc0 = kc.clone()
    out = torch.full((rows, nh * 128), 7.0, dtype=torch.bfloat16, device=dev)
    qo = out.clone()
    p = torch.full((1,), max_len, dtype=torch.long, device=dev)
    ws = torch.empty(int(L.qs_dec_attention_workspace_bytes(rows, nkv, max_len)), dtype=torch.uint8, device=dev)
    st = lib.stream_of(q)
    lib.check(L.qs_dec_qk_norm_rope(lib.ptr(q), lib.ptr(kv), lib.ptr(kv), lib.ptr(w), lib.ptr(w), lib.ptr(tab),
                                    lib.ptr(tab), lib.ptr(p), lib.ptr(qo), lib.ptr(kc), lib.ptr(vc), rows, nh, nkv, 128,
                                    max_len, 1e-6, st))
    lib.check(L.qs_dec_attention_rope(lib.ptr(q), lib.ptr(kv), lib.ptr(kv), lib.ptr(w), lib.ptr(w), lib.ptr(tab),
                                      lib.ptr(tab), lib.ptr(p), lib.ptr(kc), lib.ptr(vc), lib.ptr(out), nh * 128,
                                      lib.ptr(ws), ws.numel(), rows, nh, nkv, 128, max_len, 1e-6, 0.1, st))
    torch.cuda.synchronize()
    assert torch.equal(kc, kc0) and torch.equal(vc, kc0)
    assert (out == 7.0).all() and (qo == 7.0).all()


def test_attention_workspace_and_argument_checks(dev):
    lib, L = _lib()
    # per (row, kv head, split of 64): max and sum of 16 heads, 16 x 128 outputs
    assert L.qs_dec_attention_workspace_bytes(1, 8, 770) == 1 * 8 * math.ceil(770 / 64) * (32 + 16 * 128) * 4
    x = torch.zeros(64, dtype=torch.bfloat16, device=dev)
    pos = torch.zeros(1, dtype=torch.long, device=dev)
    # head_dim other than 128, more than 16 query heads per kv head, short workspace
    assert L.qs_dec_attention(lib.ptr(x), lib.ptr(x), lib.ptr(x), lib.ptr(pos), lib.ptr(x), 64 * 64, lib.ptr(x), 128,
                              1, 64, 8, 64, 16, 0.1, None) != 0
    assert L.qs_dec_attention(lib.ptr(x), lib.ptr(x), lib.ptr(x), lib.ptr(pos), lib.ptr(x), 64 * 128, lib.ptr(x), 1 << 20,
                              1, 64, 2, 128, 16, 0.1, None) != 0
    assert L.qs_dec_attention(lib.ptr(x), lib.ptr(x), lib.ptr(x), lib.ptr(pos), lib.ptr(x), 64 * 128, lib.ptr(x), 16,
                              1, 64, 8, 128, 16, 0.1, None) != 0
    # the same refusals with the norm + rotary inside
    X = lib.ptr(x)
    for ldo, wsb, nkv, hd in [(64 * 64, 1 << 20, 8, 64), (64 * 128, 1 << 20, 2, 128), (64 * 128, 16, 8, 128)]:
        assert L.qs_dec_attention_rope(X, X, X, X, X, X, X, lib.ptr(pos), X, X, X, ldo, X, wsb, 1, 64, nkv, hd, 16,
                                       1e-6, 0.1, None) != 0


@pytest.mark.parametrize("rows,m", [(1, 25600), (8, 25600), (3, 1536)])
def test_silu_mul(dev, rows, m):
    lib, L = _lib()
    g = torch.Generator().manual_seed(m + rows)
    gt = (torch.randn(rows, m, generator=g) * 4).bfloat16().to(dev)
    up = torch.randn(rows, m, generator=g).bfloat16().to(dev)
    out = torch.empty_like(gt)
    lib.check(L.qs_dec_silu_mul(lib.ptr(gt), lib.ptr(up), lib.ptr(out), rows, m, m, m, m, lib.stream_of(gt)))
    torch.cuda.synchronize()
    want = torch.nn.functional.silu(gt) * up
    assert _bf16_ulps(out, want) <= 1


def _lins(dev, shapes, n, seed):
    import numpy as np
    from test_gpu_linear import _rand_linear
    rng = np.random.default_rng(seed)
    return [_rand_linear(dev, rng, m, n, 1, g == 0) for g, m in enumerate(shapes)]


_PRE_SHAPES = [([8192, 1024, 1024], 5120), ([4096, 4096, 4096], 4096), ([25600, 25600], 5120), ([11008], 16384)]


@pytest.mark.parametrize("shapes,n,B", [(sh, n, B) for sh, n in _PRE_SHAPES for B in (1, 2)]
                         + [(sh, n, B) for sh, n in _PRE_SHAPES[:3] for B in (3, 8, 16)]
                         + [([1536, 2304], 3584, 8), ([4096], 11008, 8)])
@pytest.mark.parametrize("residual", [True, False])
def test_group_pre_rmsnorm_equals_separate(dev, shapes, n, B, residual):
    """RMSNorm (with the residual add) inside the grouped forward -- the
    one-launch kernel at 1-2 rows, the input-transform launch at 3-16 rows
    (n = 3584: odd factor 7; n = 11008: odd factor 43, three chunks per
    wave) -- outputs and the
    residual stream bit-identical to qs_dec_rmsnorm followed by the grouped
    forward."""
    from quipsharp_amd.quantize import forward_packed_group, pre_ok
    print(f"case: group pre rmsnorm {shapes} n={n} B={B} residual={residual}", flush=True)
    lib, L = _lib()
    g = torch.Generator().manual_seed(B + n)
    h = (torch.randn(B, n, generator=g) * 3).bfloat16().to(dev)
    d = torch.randn(B, n, generator=g).bfloat16().to(dev) if residual else None
    w = (1 + 0.1 * torch.randn(n, generator=g)).bfloat16().to(dev)
    lins = _lins(dev, shapes, n, n + len(shapes))
    h_ref, x = torch.empty_like(h), torch.empty_like(h)
    lib.check(L.qs_dec_rmsnorm(lib.ptr(h), lib.ptr(d), lib.ptr(h_ref if residual else None), lib.ptr(w), lib.ptr(x),
                               B, n, n, 1e-6, lib.stream_of(h)))
    want = forward_packed_group(x, lins)
    h_out = torch.full_like(h, 7.0)
    pre = {"kind": "rmsnorm", "delta": d, "weight": w, "h_out": h_out, "eps": 1e-6}
    assert pre_ok(h, n, pre)
    got = forward_packed_group(h, lins, pre=pre)
    torch.cuda.synchronize()
    for y, yw in zip(got, want):
        assert torch.equal(y, yw)
    assert torch.equal(h_out, h_ref if residual else h)


def test_group_pre_refused_shapes(dev):
    """Past 16 rows (the wide path), a norm wider than 16384 and an h_out
    that overlaps x are refused on the host, nothing launched."""
    from quipsharp_amd import _lib as lb
    from quipsharp_amd.quantize import pre_ok
    lib, L = _lib()
    n = 4096
    (lin,) = _lins(dev, [1024], n, 5)
    packed, su, sv, s0, s1, sc, bias = lin
    w = torch.ones(n, dtype=torch.bfloat16, device=dev)

    def call(x, pre, y):
        jobs = (lb.LinearJob * 1)()
        jobs[0] = lb.LinearJob(packed.codes0.data_ptr(), None, 1024, su.data_ptr(), sv.data_ptr(), 1, None, s0, s1, sc,
                               bias.data_ptr(), y.data_ptr(), 1024, 0)
        ws = torch.zeros(1 << 22, dtype=torch.uint8, device=dev)
        return L.qs_linear_forward_group_pre(lb.ptr(x), n, x.shape[0], n, 1, None, 1, jobs, pre, lb.QS_DTYPE_BF16,
                                             lb.ptr(ws), ws.numel(), lb.stream_of(x))

    x3 = torch.randn(17, n, device=dev).bfloat16()
    y3 = torch.full((17, 1024), 5.0, dtype=torch.bfloat16, device=dev)
    op = lb.PreOp(lb.QS_PREOP_RMSNORM, None, n, lb.ptr(w), None, n, 1e-6)
    assert call(x3, op, y3) == 3 and not pre_ok(x3, n, {"kind": "rmsnorm"})
    x1 = torch.randn(1, n, device=dev).bfloat16()
    y1 = torch.full((1, 1024), 5.0, dtype=torch.bfloat16, device=dev)
    op = lb.PreOp(lb.QS_PREOP_RMSNORM, None, n, lb.ptr(w), lb.ptr(x1), n, 1e-6)  # h_out == x
    assert call(x1, op, y1) == 1 and b"overlaps" in L.qs_last_error()
    torch.cuda.synchronize()
    assert bool((y3 == 5.0).all()) and bool((y1 == 5.0).all())
