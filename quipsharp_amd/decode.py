"""Greedy-decode harness for a full quantized decoder (Qwen3-32B shape by
default): every decoder linear is a QuantizedLinear with random E8P codes,
the rest of the model (embeddings, norms, rotary tables, lm_head) is the
transformers implementation in bf16 with random weights.  Built on the meta
device and materialized on the GPU, so the 32B-parameter model never exists
densely.  Decoding runs through StaticDecoder (static bf16 KV cache, device
positions, the decode step's own kernels around the quantized linears) so
that each step is one HIP-graph replay.  Reports
prefill time, decode tok/s and, per decoder linear of the first layer, the
forward time and HBM GB/s at each batch size.

    python -m quipsharp_amd.decode --batch 1 8 --prompt 512 --new 256
"""
import argparse
import json
import time

import torch
from torch import nn

from .architectures import get_decoder_layers, get_linear_groups
from .checkpoint import (QuantizedLinear, build_codebook, grouped_forward, grouped_forward_pre,
                         link_sibling_linears)
from .hadamard import is_pow2, kron_factor, rademacher

QWEN3_32B = dict(hidden_size=5120, intermediate_size=25600, num_hidden_layers=64, num_attention_heads=64,
                 num_key_value_heads=8, head_dim=128, vocab_size=151936, max_position_embeddings=40960,
                 rms_norm_eps=1e-6, tie_word_embeddings=False)


def _random_qlinear(lin, device, gen, cpu_gen, scale=0.0135):
    n, m = lin.in_features, lin.out_features
    kind = "rht" if is_pow2(n) and is_pow2(m) else "krht"
    if kind == "krht" and (kron_factor(n) is None or kron_factor(m) is None):
        raise ValueError(f"no transform for a {m} x {n} linear")
    q = QuantizedLinear(n, m, 8, kind, has_bias=getattr(lin, "bias", None) is not None)
    q = q.to(device)
    with torch.no_grad():
        q.codes.copy_(torch.randint(-32768, 32768, q.codes.shape, generator=gen, device=device, dtype=torch.int32)
                      .to(torch.int16))
        q.scale.fill_(scale)
        q.su.copy_(rademacher(m, device=device, generator=cpu_gen))
        q.sv.copy_(rademacher(n, device=device, generator=cpu_gen))
        if q.bias is not None:
            q.bias.zero_()
    return q


def random_quantized_model(config, device="cuda", seed=0):
    """transformers causal LM of ``config`` with every decoder linear replaced
    by a random-code QuantizedLinear (linear discovery as
    architectures.get_linear_groups) and random bf16 for the rest."""
    from transformers import AutoModelForCausalLM
    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16)
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu_gen = torch.Generator().manual_seed(seed)
    codebook, _ = build_codebook("2bit", device, seed)
    for i, layer in enumerate(get_decoder_layers(model)):
        for group in get_linear_groups(layer, i):
            for name, lin in group:
                parent_name, _, attr = name.rpartition(".")
                parent = layer.get_submodule(parent_name)
                q = _random_qlinear(lin, device, gen, cpu_gen)
                q.codebook = codebook
                setattr(parent, attr, q)
    # everything still on the meta device gets fresh storage on the GPU
    for mod in model.modules():
        if hasattr(mod, "inv_freq") and getattr(mod, "inv_freq").is_meta:
            fresh = type(mod)(config=mod.config)
            for k, v in fresh.named_buffers(recurse=False):
                setattr(mod, k, v.to(device))
            if hasattr(fresh, "attention_scaling"):
                mod.attention_scaling = fresh.attention_scaling
            continue
        for k, p in list(mod.named_parameters(recurse=False)):
            if p.is_meta:
                if "norm" in type(mod).__name__.lower():
                    t = torch.ones(p.shape, dtype=p.dtype, device=device)
                else:
                    t = torch.randn(p.shape, generator=gen, dtype=torch.float32, device=device).mul_(0.02)
                    t = t.to(p.dtype)
                setattr(mod, k, nn.Parameter(t, requires_grad=False))
        for k, b in list(mod.named_buffers(recurse=False)):
            if b is not None and b.is_meta:
                setattr(mod, k, torch.zeros(b.shape, dtype=b.dtype, device=device))
    model.eval()
    link_sibling_linears(model)
    return model


@torch.no_grad()
def greedy_decode(model, prompt_ids, new_tokens):
    """Prefill ``prompt_ids`` (B, P), then ``new_tokens`` greedy steps with a
    KV cache.  Returns (tokens (B, new_tokens), prefill s, decode s)."""
    from transformers import DynamicCache
    cache = DynamicCache()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = model(input_ids=prompt_ids, past_key_values=cache, use_cache=True)
    nxt = out.logits[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    toks = [nxt]
    for _ in range(new_tokens - 1):
        out = model(input_ids=nxt, past_key_values=cache, use_cache=True)
        nxt = out.logits[:, -1].argmax(-1, keepdim=True)
        toks.append(nxt)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    return torch.cat(toks, 1), t1 - t0, t2 - t1


class StaticDecoder:
    """A graph-capturable greedy-decode step for Qwen3-style decoders built on
    the transformers modules of ``model`` (embeddings, RMSNorm and q/k-norm
    weights, rotary tables, lm_head) and its QuantizedLinear layers, with a
    static bf16 KV cache of ``max_len`` positions per layer and the position
    passed as a device tensor, so one decode step can be captured once and
    replayed.

    A decode step (one new token per row) runs the layer's own kernels
    (csrc/qs_decoder.hip): q/k norm plus rotary embedding plus the cache
    write in one launch, attention over the filled cache prefix only (splits
    of 64 positions and a combine launch), SiLU * up; q/k/v and gate/up each
    go through one grouped quantized-linear launch that, at one row, also
    does the residual add and the RMSNorm before it
    (checkpoint.grouped_forward_pre; at more rows the norm runs on its own
    launch first).  The prompt
    (several tokens per row) runs transformers' modules with the same bf16
    cache (attention in fp32)."""

    def __init__(self, model, batch, max_len):
        from . import _lib
        cfg = model.config
        self.model = model
        self.layers = get_decoder_layers(model)
        self.B, self.max_len = batch, max_len
        self.nh, self.nkv, self.hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.hidden = cfg.hidden_size
        self.eps = float(cfg.rms_norm_eps)
        self.scale = self.hd ** -0.5
        dev = model.lm_head.weight.device
        self.dev = dev
        bf = torch.bfloat16
        self.k = [torch.zeros(batch, self.nkv, max_len, self.hd, device=dev, dtype=bf) for _ in self.layers]
        self.v = [torch.zeros(batch, self.nkv, max_len, self.hd, device=dev, dtype=bf) for _ in self.layers]
        self.kpos = torch.arange(max_len, device=dev)
        # rotary tables of every cache position, as transformers computes them
        m = model.model
        with torch.no_grad():
            cos, sin = m.rotary_emb(torch.zeros(1, 1, self.hidden, device=dev, dtype=bf), self.kpos[None])
        self.cos, self.sin = cos[0].to(bf).contiguous(), sin[0].to(bf).contiguous()
        L = _lib.lib()
        self._L, self._lib = L, _lib
        nbytes = L.qs_dec_attention_workspace_bytes(batch, self.nkv, max_len)
        self.attn_ws = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)
        self.fused_ok = self.hd == 128 and self.nh % self.nkv == 0 and self.nh // self.nkv <= 16 \
            and self.hidden % 8 == 0

    def _weight(self, mod):
        w = mod.weight
        if w.dtype != torch.bfloat16 or not w.is_contiguous():
            raise TypeError("the decode step takes bf16 norm weights")
        return w

    @torch.no_grad()
    def step(self, ids, pos):
        """Logits of the last position; ids (B, q), pos (q,) int64 positions."""
        if ids.shape[1] == 1 and self.fused_ok:
            return self._decode_step(ids, pos)
        return self._prompt_step(ids, pos)

    def _prompt_step(self, ids, pos):
        from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
        import torch.nn.functional as F
        m = self.model.model
        B, q = ids.shape
        h = m.embed_tokens(ids)
        cos, sin = m.rotary_emb(h, pos.unsqueeze(0).expand(B, -1))
        mask = self.kpos[None, :] <= pos[:, None]  # (q, max_len): key j visible to query at pos_i iff j <= pos_i
        for i, L in enumerate(self.layers):
            a = L.self_attn
            x = L.input_layernorm(h)
            qo, ko, vo = grouped_forward(x, [a.q_proj, a.k_proj, a.v_proj])
            qs = a.q_norm(qo.view(B, q, self.nh, self.hd)).transpose(1, 2)
            ks = a.k_norm(ko.view(B, q, self.nkv, self.hd)).transpose(1, 2)
            vs = vo.view(B, q, self.nkv, self.hd).transpose(1, 2)
            qs, ks = apply_rotary_pos_emb(qs, ks, cos, sin)
            self.k[i].index_copy_(2, pos, ks.to(self.k[i].dtype))
            self.v[i].index_copy_(2, pos, vs.to(self.v[i].dtype))
            o = F.scaled_dot_product_attention(qs.float(), self.k[i].float(), self.v[i].float(), attn_mask=mask,
                                               enable_gqa=True)
            h = h + a.o_proj(o.transpose(1, 2).reshape(B, q, self.nh * self.hd).to(h.dtype))
            x = L.post_attention_layernorm(h)
            go, uo = grouped_forward(x, [L.mlp.gate_proj, L.mlp.up_proj])
            h = h + L.mlp.down_proj(L.mlp.act_fn(go) * uo)
        return self.model.lm_head(m.norm(h[:, -1:]))[:, -1]

    def _decode_step(self, ids, pos):
        L, lib = self._L, self._lib
        m = self.model.model
        B = ids.shape[0]
        H, nh, nkv, hd = self.hidden, self.nh, self.nkv, self.hd
        stream = lib.stream_of(ids)
        vp = lib.ptr
        h = m.embed_tokens(ids).reshape(B, H)
        if h.dtype != torch.bfloat16:
            raise TypeError("the decode step runs bf16 models")
        h = h.contiguous()
        # the residual stream alternates between two buffers: a norm inside a
        # grouped launch reads h + delta while one work-group writes the sum
        h_alt = torch.empty_like(h)
        attn = torch.empty(B, nh * hd, dtype=torch.bfloat16, device=h.device)
        delta = None
        for i, Ly in enumerate(self.layers):
            a = Ly.self_attn
            # residual add + input norm inside the q/k/v launch (one row; on
            # their own launch otherwise)
            qo, ko, vo = grouped_forward_pre(h, [a.q_proj, a.k_proj, a.v_proj],
                                             {"kind": "rmsnorm", "delta": delta, "h_out": h_alt, "eps": self.eps,
                                              "weight": self._weight(Ly.input_layernorm)})
            h, h_alt = h_alt, h
            # q/k norm, rotary and the cache write inside the attention's launches
            lib.check(L.qs_dec_attention_rope(vp(qo.contiguous()), vp(ko.contiguous()), vp(vo.contiguous()),
                                              vp(self._weight(a.q_norm)), vp(self._weight(a.k_norm)), vp(self.cos),
                                              vp(self.sin), vp(pos), vp(self.k[i]), vp(self.v[i]), vp(attn), nh * hd,
                                              vp(self.attn_ws), self.attn_ws.numel(), B, nh, nkv, hd, self.max_len,
                                              self.eps, self.scale, stream))
            o = a.o_proj(attn).contiguous()
            go, uo = grouped_forward_pre(h, [Ly.mlp.gate_proj, Ly.mlp.up_proj],
                                         {"kind": "rmsnorm", "delta": o, "h_out": h_alt, "eps": self.eps,
                                          "weight": self._weight(Ly.post_attention_layernorm)})
            h, h_alt = h_alt, h
            go, uo = go.contiguous(), uo.contiguous()
            act = torch.empty_like(go)
            inter = go.shape[-1]
            lib.check(L.qs_dec_silu_mul(vp(go), vp(uo), vp(act), B, inter, inter, inter, inter, stream))
            delta = Ly.mlp.down_proj(act).contiguous()
        x = torch.empty_like(h)
        lib.check(L.qs_dec_rmsnorm(vp(h), vp(delta), vp(h), vp(self._weight(m.norm)), vp(x), B, H, H, self.eps, stream))
        return self.model.lm_head(x)


@torch.no_grad()
def greedy_decode_static(model, prompt_ids, new_tokens, use_graph=True):
    """Prefill and greedy decode with StaticDecoder; each decode step replayed
    from one HIP graph unless use_graph=False.  Returns (tokens, prefill s,
    decode s)."""
    B, P = prompt_ids.shape
    dev = prompt_ids.device
    dec = StaticDecoder(model, B, P + new_tokens + 2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = dec.step(prompt_ids, torch.arange(P, device=dev)).argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    pos = torch.full((1,), P, dtype=torch.long, device=dev)
    toks = [tok.clone()]
    if not use_graph:
        for _ in range(new_tokens - 1):
            tok = dec.step(tok, pos).argmax(-1, keepdim=True)
            pos.add_(1)
            toks.append(tok)
        torch.cuda.synchronize()
        return torch.cat(toks, 1), t1 - t0, time.perf_counter() - t1
    # warm-up (writes position P with the right token, as the first replay will), then capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            dec.step(tok, pos)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        nxt = dec.step(tok, pos).argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for _ in range(new_tokens - 1):
        graph.replay()
        tok.copy_(nxt)
        pos.add_(1)
        toks.append(nxt.clone())
    torch.cuda.synchronize()
    return torch.cat(toks, 1), t1 - t0, time.perf_counter() - t2


def linear_bytes(m, n, B):
    """Algorithmic HBM bytes of one quantized-linear call: 2-byte codes per 8
    weights, bf16 activations in and out, 1-bit signs, fp16 scale."""
    return m * n // 8 * 2 + 2 * B * (n + m) + -(-(m + n) // 8) + 2


def linear_gbps(model, batches, reps=20):
    """Per-linear forward time and HBM GB/s (algorithmic bytes) for the
    decoder linears of the first layer, at each batch size: ``reps`` calls of
    the module captured in one HIP graph, replayed and timed with events."""
    layer = get_decoder_layers(model)[0]
    out = []
    dev = next(model.parameters()).device
    for group in get_linear_groups(layer, 0):
        for name, lin in group:
            n, m = lin.in_features, lin.out_features
            for B in batches:
                x = torch.randn(B, n, device=dev).bfloat16()
                with torch.no_grad():
                    lin(x)  # workspace, packed codes
                    torch.cuda.synchronize()
                    s = torch.cuda.Stream(device=dev)
                    s.wait_stream(torch.cuda.current_stream(dev))
                    with torch.cuda.stream(s):
                        lin(x)
                    torch.cuda.current_stream(dev).wait_stream(s)
                    torch.cuda.synchronize()
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g):
                        for _ in range(reps):
                            lin(x)
                    g.replay()
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(5):
                        g.replay()
                    e1.record()
                    torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / (5 * reps)
                nb = linear_bytes(m, n, B)
                out.append({"linear": name, "m": m, "n": n, "batch": B, "us": round(us, 2),
                            "GBps": round(nb / (us * 1e-6) / 1e9, 1)})
                del g
    return out


def _graph_time(fn, replays=10):
    """Median ms of one replay of ``fn`` captured in a HIP graph (after a
    warm-up call outside capture and two warm-up replays)."""
    import statistics
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    ev[0].record()
    for i in range(replays):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    ms = statistics.median(ev[i].elapsed_time(ev[i + 1]) for i in range(replays))
    del g
    return ms


@torch.no_grad()
def linears_step_ms(model, batch):
    """ms of the decoder linears alone for one decode step of ``batch`` rows,
    in StaticDecoder's order and call pattern (q/k/v grouped, o, gate/up
    grouped, down; each layer's input the previous layer's output), replayed
    from a HIP graph."""
    layers = get_decoder_layers(model)
    dev = next(model.parameters()).device
    h = torch.randn(batch, model.config.hidden_size, device=dev).bfloat16()

    def run():
        x = h
        for L in layers:
            a = L.self_attn
            qo, _, _ = grouped_forward(x, [a.q_proj, a.k_proj, a.v_proj])
            o = a.o_proj(qo)
            go, _ = grouped_forward(o, [L.mlp.gate_proj, L.mlp.up_proj])
            x = L.mlp.down_proj(go)
        return x
    return _graph_time(run)


@torch.no_grad()
def linear_gbps_rotated(model, batch):
    """Per decoder linear (q, k, v, o, gate, up, down): us and GB/s
    (algorithmic bytes) of one call, from a HIP graph that calls that linear
    of every decoder layer in turn, so the codes read per replay (for gate /
    up, 64 x 33 MB) far exceed the 256 MB Infinity Cache."""
    layers = get_decoder_layers(model)
    dev = next(model.parameters()).device
    out = []
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
        mods = [getattr(L.self_attn if name[0] in "qkvo" else L.mlp, name) for L in layers]
        n, m = mods[0].in_features, mods[0].out_features
        x = torch.randn(batch, n, device=dev).bfloat16()
        # _forward_one: this linear alone (a linked q or gate called under
        # capture would run its whole group)
        ms = _graph_time(lambda: [mod._forward_one(x) for mod in mods])
        us = ms * 1e3 / len(mods)
        out.append({"linear": name, "m": m, "n": n, "batch": batch, "us": round(us, 2),
                    "GBps": round(linear_bytes(m, n, batch) / (us * 1e-6) / 1e9, 1)})
    return out


def measure_decode(layers=64, batches=(1, 8), prompt=512, new=64, device="cuda:0"):
    """The Qwen3-32B-shaped greedy decode of ``new`` tokens after a ``prompt``
    -token random prompt, per batch size: prefill s, decode tok/s and ms per
    step (graph-replayed steps), the decoder linears' ms per step and the
    rest, and per-linear GB/s rotated over all layers."""
    from transformers import Qwen3Config
    cfg = Qwen3Config(**dict(QWEN3_32B, num_hidden_layers=layers))
    dev = torch.device(device)
    t0 = time.perf_counter()
    model = random_quantized_model(cfg, dev)
    torch.cuda.synchronize()
    res = {"model": "Qwen3-32B shape (64 layers, hidden 5120, intermediate 25600, 64 q / 8 kv heads, "
                    "vocab 151936), random init, every decoder linear E8P 2-bit", "layers": layers,
           "code_bytes": sum(m.codes.numel() * 2 for m in model.modules() if isinstance(m, QuantizedLinear)),
           "build_s": round(time.perf_counter() - t0, 1), "prompt": prompt, "new_tokens": new, "runs": []}
    for B in batches:
        g = torch.Generator().manual_seed(B)
        ids = torch.randint(0, cfg.vocab_size, (B, prompt), generator=g).to(dev)
        greedy_decode(model, ids[:, :16], 4)  # warm-up
        toks, pre_s, dec_s = greedy_decode_static(model, ids, new)
        steps = new - 1
        step_ms = 1e3 * dec_s / steps
        lin_ms = linears_step_ms(model, B)
        res["runs"].append({"batch": B, "prefill_s": round(pre_s, 3), "tok_per_s": round(B * steps / dec_s, 2),
                            "ms_per_step": round(step_ms, 3), "linears_ms_per_step": round(lin_ms, 3),
                            "other_ms_per_step": round(step_ms - lin_ms, 3),
                            "linears_GBps": round(res["code_bytes"] / (lin_ms * 1e-3) / 1e9, 1),
                            "per_linear": linear_gbps_rotated(model, B), "first_tokens": toks[0, :8].tolist()})
    del model
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--batch", type=int, nargs="+", default=[1, 8])
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--new", type=int, default=256)
    ap.add_argument("--eager", action="store_true", help="decode steps launched eagerly (no HIP graph)")
    args = ap.parse_args()
    from transformers import Qwen3Config
    cfg = Qwen3Config(**dict(QWEN3_32B, num_hidden_layers=args.layers))
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    model = random_quantized_model(cfg, dev)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    code_bytes = sum(m.codes.numel() * 2 for m in model.modules() if isinstance(m, QuantizedLinear))
    res = {"model": "Qwen3-32B shape (random init, E8P 2-bit decoder linears)", "layers": args.layers,
           "code_bytes": code_bytes, "build_s": round(build_s, 1), "runs": []}
    for B in args.batch:
        g = torch.Generator().manual_seed(B)
        ids = torch.randint(0, cfg.vocab_size, (B, args.prompt), generator=g).to(dev)
        greedy_decode(model, ids[:, :16], 4)  # warm-up
        toks, pre_s, dec_s = greedy_decode_static(model, ids, args.new, use_graph=not args.eager)
        steps = args.new - 1
        res["runs"].append({"batch": B, "graph": not args.eager, "prefill_s": round(pre_s, 3), "decode_s": round(dec_s, 3),
                            "tok_per_s": round(B * steps / dec_s, 2), "ms_per_step": round(1e3 * dec_s / steps, 3),
                            "first_tokens": toks[0, :8].tolist()})
    res["per_linear"] = linear_gbps(model, args.batch)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
