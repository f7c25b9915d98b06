"""Writes the golden fixtures in tests/golden/ by running numbersletter/quipsharp
on the CPU of the development container.

Run by hand (never by the tests, never on a GPU box, which has no copy of the
reference):

    python tests/golden/make_golden.py /root/reference

What it pins that closed forms and brute force cannot:
  * E8P encode tie-breaking and E8 1-bit / RVQ codes at bit level
    (quipsharp/codebooks/e8p.py:104-171, e8_1bit.py:80-83, rvq.py:69-80);
  * the fitted codebook scales of build_codebook (checkpoint.py:60-77,
    rvq.py:28-66), which only the reference's own RNG draw and sweep fix;
  * fwht outputs at bit level (hadamard.py:17-40);
  * quantize_linear end to end on this CPU/MKL, with every target handed to
    the codebook recorded so encode parity can be checked teacher-forced
    (quantize.py:48-104, ldlq.py:97-141);
  * linear_forward on given codes (quantize.py:116-124);
  * the RFFT transform (rfft.py:37-60), for the compat transform.
Outputs are small .npz/.json files; inputs are stored with the outputs.
"""
import hashlib
import json
import os
import sys

import numpy as np

OUT = os.path.dirname(os.path.abspath(__file__))


def main(ref_root):
    sys.path.insert(0, ref_root)
    import torch
    from quipsharp.codebooks import e8p
    from quipsharp.codebooks.e8_1bit import E8OneBitCodebook, build_table
    from quipsharp.rvq import RVQStage, rvq_quantize
    from quipsharp.quantize import (quantize_linear, linear_forward, dequantize_linear,
                                    RVQCodebookAdapter, QuantizedLayer)
    from quipsharp.incoherence import IncoherenceSigns
    from quipsharp.hadamard import fwht
    from quipsharp.checkpoint import build_codebook
    from quipsharp.ldlq import block_ldl
    from quipsharp.rfft import to_transformed_space, from_transformed_space, random_phase

    torch.set_num_threads(8)
    cb = e8p.E8PCodebook()
    onebit = E8OneBitCodebook()
    abs_table = cb.abs_table.numpy().copy()
    table1 = build_table().numpy().copy()

    # ---- tables + full decode hash ------------------------------------------
    all_codes = torch.arange(65536, dtype=torch.int64)
    dec_all = cb.dequantize(all_codes).numpy().astype(np.float32)
    np.savez_compressed(os.path.join(OUT, "tables.npz"), e8p_abs=abs_table, e81=table1,
                        e8p_decode_all_sha256=np.frombuffer(
                            hashlib.sha256(dec_all.tobytes()).digest(), np.uint8))

    # ---- encode inputs --------------------------------------------------------
    g = torch.Generator().manual_seed(1234)
    parts = []
    for sigma in (0.5, 1.0, 2.0):
        parts.append(torch.randn(1536, 8, generator=g) * sigma)
    parts.append(torch.randn(256, 8, generator=g) * 10.0)     # far outside the ball
    parts.append(torch.randn(256, 8, generator=g) * 1e-3)     # near zero
    parts.append(torch.zeros(8, 8))                           # exact ties across shifts
    cw = cb.dequantize(torch.randint(0, 65536, (256,), generator=g))
    parts.append(cw)                                          # exact codewords
    cw2 = cb.dequantize(torch.randint(0, 65536, (256,), generator=g))
    parts.append((cw + cw2) * 0.5)                            # midpoints of codeword pairs
    parts.append(cw - torch.where(torch.rand(256, 1, generator=g) < 0.5, 0.25, -0.25))  # unshifted lattice pts
    q = torch.randint(-8, 9, (256, 8), generator=g).float() * 0.25  # quarter grid: many ties
    parts.append(q)
    X = torch.cat(parts).float().contiguous()
    vals, codes = cb.quantize(X)
    assert torch.equal(cb.dequantize(codes), vals)
    vals1, idx1 = onebit.quantize(X)
    np.savez_compressed(os.path.join(OUT, "encode.npz"), x=X.numpy(),
                        e8p_code=codes.numpy().astype(np.uint16),
                        e81_idx=idx1.numpy().astype(np.uint8))

    # ---- RVQ with fixed stage scales -----------------------------------------
    rvq = {}
    for name, stages in (("rvq3", [RVQStage(cb, 1.03), RVQStage(onebit, 0.47)]),
                         ("rvq4", [RVQStage(cb, 1.03), RVQStage(cb, 0.29)])):
        tv, tc = rvq_quantize(X, stages)
        rvq[name + "_codes"] = torch.stack(tc).numpy().astype(np.int32)
        rvq[name + "_sha256"] = np.frombuffer(hashlib.sha256(tv.numpy().tobytes()).digest(), np.uint8)
    np.savez_compressed(os.path.join(OUT, "rvq.npz"), **rvq)

    # ---- fitted scales --------------------------------------------------------
    scales, books = {}, {}
    for bits in ("2bit", "3bit", "4bit"):
        c, s = build_codebook(bits, "cpu", seed=0)
        books[bits] = (c, s)
        scales[bits] = {"scale": s}
        if bits != "2bit":
            scales[bits]["stage_scales"] = [st.scale for st in c.stages]
    with open(os.path.join(OUT, "scales.json"), "w") as f:
        json.dump(scales, f, indent=2)

    # ---- fwht -----------------------------------------------------------------
    fw = {}
    g = torch.Generator().manual_seed(7)
    for k in range(0, 15):
        n = 1 << k
        rows = 2 if n <= 4096 else 1
        x = torch.randn(rows, n, generator=g)
        fw[f"x{n}"] = x.numpy()
        fw[f"y{n}"] = fwht(x, dim=-1).numpy()
    xm = torch.randn(64, 24, generator=g)
    fw["xdim0"] = xm.numpy()
    fw["ydim0"] = fwht(xm, dim=0).numpy()
    np.savez_compressed(os.path.join(OUT, "fwht.npz"), **fw)

    # ---- quantize_linear end to end (teacher-forced targets recorded) --------
    def run_quantize(m, n, codebook, cb_scale, seed):
        gg = torch.Generator().manual_seed(seed)
        W = torch.randn(m, n, generator=gg) * 0.02
        Xc = torch.randn(4 * n, n, generator=gg)
        H = Xc.T @ Xc / (4 * n)
        xin = torch.randn(3, n, generator=gg)
        calls = []

        class Rec:
            def quantize(self, t):
                v, c = codebook.quantize(t)
                calls.append((t.clone(), c.clone()))
                return v, c

            def dequantize(self, c):
                return codebook.dequantize(c)

        torch.manual_seed(0)
        layer, what_q = quantize_linear(W, H, Rec(), g=8, damping=1e-2,
                                        codebook_scale=cb_scale, tune_iters=10)
        y = linear_forward(xin, layer, codebook)
        deq = dequantize_linear(layer, codebook)
        assert torch.allclose(deq, what_q)
        return dict(W=W.numpy(), H=H.numpy(), x=xin.numpy(), y=y.numpy(),
                    codes=layer.codes.numpy().astype(np.int32), what_q=what_q.numpy(),
                    su=layer.signs.su.numpy(), sv=layer.signs.sv.numpy(),
                    layer_scale=np.float64(layer.scale),
                    targets=torch.stack([c[0] for c in calls]).numpy(),
                    target_codes=torch.stack([c[1] for c in calls]).numpy().astype(np.int32))

    cb2, s2 = books["2bit"]
    np.savez_compressed(os.path.join(OUT, "quantize2.npz"), **run_quantize(32, 128, cb2, s2, 11))
    cb3, s3 = books["3bit"]
    np.savez_compressed(os.path.join(OUT, "quantize3.npz"), **run_quantize(16, 64, cb3, s3, 12))

    # ---- linear_forward on random codes --------------------------------------
    lf = {}
    g = torch.Generator().manual_seed(99)
    for name, (m, n, stages) in (("e8p", (256, 512, 1)), ("rvq3", (128, 256, 2))):
        T = n // 8
        if stages == 1:
            codes = torch.randint(0, 65536, (m, T), generator=g)
            book = cb
        else:
            codes = torch.stack([torch.randint(0, 65536, (m, T), generator=g),
                                 torch.randint(0, 256, (m, T), generator=g)])
            book = RVQCodebookAdapter([RVQStage(cb, 1.03), RVQStage(onebit, 0.47)])
        su = torch.randint(0, 2, (m,), generator=g).float() * 2 - 1
        sv = torch.randint(0, 2, (n,), generator=g).float() * 2 - 1
        scale = float(np.float32(0.0135))
        layer = QuantizedLayer(codes=codes, signs=IncoherenceSigns(su=su, sv=sv), g=8,
                               shape=(m, n), scale=scale)
        x = torch.randn(4, n, generator=g)
        lf[name + "_codes"] = codes.numpy().astype(np.int32)
        lf[name + "_su"] = su.numpy()
        lf[name + "_sv"] = sv.numpy()
        lf[name + "_scale"] = np.float32(scale)
        lf[name + "_x"] = x.numpy()
        lf[name + "_y"] = linear_forward(x, layer, book).numpy()
        lf[name + "_deq"] = dequantize_linear(layer, book).numpy()
    np.savez_compressed(os.path.join(OUT, "linear.npz"), **lf)

    # ---- block LDL ------------------------------------------------------------
    g = torch.Generator().manual_seed(5)
    A = torch.randn(64, 64, generator=g)
    Hs = A @ A.T + torch.eye(64)
    L, D = block_ldl(Hs, 8, damping=0.0)
    np.savez_compressed(os.path.join(OUT, "ldl.npz"), H=Hs.numpy(), L=L.numpy(), D=D.numpy())

    # ---- RFFT -----------------------------------------------------------------
    g = torch.Generator().manual_seed(3)
    ph = random_phase(72, generator=g)
    x = torch.randn(3, 144, generator=g)
    np.savez_compressed(os.path.join(OUT, "rfft.npz"), phase=torch.view_as_real(ph).numpy(), x=x.numpy(),
                        fwd=to_transformed_space(x, ph).numpy(), inv=from_transformed_space(x, ph).numpy())
    print("golden fixtures written to", OUT)


def c1_full(ref_root):
    """The full-size 4096x4096 E8P 2-bit quantize with the reference's recipe:
    W = 0.02 N(0,1), H = X^T X / 2048 with X in R^{2048x4096}, x in R^4096,
    all drawn from Generator().manual_seed(0) in that order; torch.manual_seed(0)
    right before quantize_linear (su then sv from the global CPU RNG);
    build_codebook("2bit", "cpu", 0); damping 1e-2, tune_iters 10
    (quipsharp/quantize.py:48-104, ldlq.py:97-141, checkpoint.py:56-77).

    Writes c1_full.npz: every code (u16 [4096, 512]) with its SHA-256,
    layer_scale, y = linear_forward(x), the signs (int8), and the reference's
    own relative proxy loss tr(E H E^T) / tr(W H W^T) in the transformed basis.
    Takes ~20 minutes on 8 cores."""
    import time
    sys.path.insert(0, ref_root)
    import torch
    from quipsharp.checkpoint import build_codebook
    from quipsharp.quantize import quantize_linear, linear_forward
    from quipsharp.incoherence import incoherence_process

    torch.set_num_threads(int(os.environ.get("C1_THREADS", "8")))
    g = torch.Generator().manual_seed(0)
    W = torch.randn(4096, 4096, generator=g) * 0.02
    X = torch.randn(2048, 4096, generator=g)
    H = X.T @ X / 2048
    x = torch.randn(4096, generator=g)
    cb, s = build_codebook("2bit", "cpu", 0)
    t0 = time.time()
    torch.manual_seed(0)
    layer, what_q = quantize_linear(W, H, cb, g=8, damping=1e-2, codebook_scale=s, tune_iters=10)
    t_q = time.time() - t0
    y = linear_forward(x, layer, cb)
    # proxy loss in the transformed basis (the basis BlockLDLQ minimizes in)
    Hd = H + 1e-2 * H.diagonal().mean() * torch.eye(4096)
    torch.manual_seed(0)
    what, hhat, signs = incoherence_process(W, Hd)
    assert torch.equal(signs.su, layer.signs.su) and torch.equal(signs.sv, layer.signs.sv)
    E = (what_q - what).double()
    Wd = what.double()
    Hh = hhat.double()
    proxy_rel = (torch.trace(E @ Hh @ E.T) / torch.trace(Wd @ Hh @ Wd.T)).item()
    codes = layer.codes.numpy().astype(np.uint16)
    np.savez_compressed(os.path.join(OUT, "c1_full.npz"), codes=codes,
                        codes_sha256=np.frombuffer(hashlib.sha256(codes.tobytes()).digest(), np.uint8),
                        layer_scale=np.float64(layer.scale), y=y.numpy(),
                        su=layer.signs.su.numpy().astype(np.int8),
                        sv=layer.signs.sv.numpy().astype(np.int8),
                        proxy_rel=np.float64(proxy_rel), quantize_seconds=np.float64(t_q),
                        threads=np.int32(torch.get_num_threads()))
    print(f"c1_full.npz written: quantize {t_q:.0f} s, proxy_rel {proxy_rel:.5e}", flush=True)


def c1_full_3bit(ref_root):
    """The C1 recipe (same W, H, x draws and torch.manual_seed(0) before
    quantize_linear) with the 3-bit RVQ codebook: build_codebook("3bit",
    "cpu", 0), i.e. [E8P, E8 1-bit] stages with their fitted scales and the
    RVQ's own input scale (checkpoint.py:60-77, rvq.py:69-88,
    quantize.py:48-104).

    Writes c1_full_3bit.npz: stage-1 codes (u16 [4096, 512]) and stage-2
    codes (u8 [4096, 512]) with their SHA-256, layer_scale, the codebook
    scales, y = linear_forward(x), the signs and the relative proxy loss
    tr(E H E^T) / tr(W H W^T) in the transformed basis."""
    import time
    sys.path.insert(0, ref_root)
    import torch
    from quipsharp.checkpoint import build_codebook
    from quipsharp.quantize import quantize_linear, linear_forward
    from quipsharp.incoherence import incoherence_process

    torch.set_num_threads(int(os.environ.get("C1_THREADS", "8")))
    g = torch.Generator().manual_seed(0)
    W = torch.randn(4096, 4096, generator=g) * 0.02
    X = torch.randn(2048, 4096, generator=g)
    H = X.T @ X / 2048
    x = torch.randn(4096, generator=g)
    cb, s = build_codebook("3bit", "cpu", 0)
    t0 = time.time()
    torch.manual_seed(0)
    layer, what_q = quantize_linear(W, H, cb, g=8, damping=1e-2, codebook_scale=s, tune_iters=10)
    t_q = time.time() - t0
    y = linear_forward(x, layer, cb)
    Hd = H + 1e-2 * H.diagonal().mean() * torch.eye(4096)
    torch.manual_seed(0)
    what, hhat, signs = incoherence_process(W, Hd)
    assert torch.equal(signs.su, layer.signs.su) and torch.equal(signs.sv, layer.signs.sv)
    E = (what_q - what).double()
    Wd = what.double()
    Hh = hhat.double()
    proxy_rel = (torch.trace(E @ Hh @ E.T) / torch.trace(Wd @ Hh @ Wd.T)).item()
    assert layer.codes.shape == (2, 4096, 512)
    c0 = layer.codes[0].numpy().astype(np.uint16)
    c1 = layer.codes[1].numpy().astype(np.uint8)
    assert np.array_equal(c1.astype(np.int64), layer.codes[1].numpy())
    sha = lambda a: np.frombuffer(hashlib.sha256(a.tobytes()).digest(), np.uint8)
    np.savez_compressed(os.path.join(OUT, "c1_full_3bit.npz"), codes0=c0, codes1=c1,
                        codes0_sha256=sha(c0), codes1_sha256=sha(c1),
                        layer_scale=np.float64(layer.scale), codebook_scale=np.float64(s),
                        stage_scales=np.array([st.scale for st in cb.stages], np.float64), y=y.numpy(),
                        su=layer.signs.su.numpy().astype(np.int8),
                        sv=layer.signs.sv.numpy().astype(np.int8),
                        proxy_rel=np.float64(proxy_rel), quantize_seconds=np.float64(t_q),
                        threads=np.int32(torch.get_num_threads()))
    print(f"c1_full_3bit.npz written: quantize {t_q:.0f} s, proxy_rel {proxy_rel:.5e}", flush=True)


def ref_checkpoint(ref_root):
    """A checkpoint written by the reference's own save path
    (quipsharp/checkpoint.py:149-186, driven as scripts/quantize_model.py:72-126
    drives it): a one-layer Llama-shaped model, hidden 256 (power of two:
    "rht" layers, with q/k/v/o biases) and intermediate 384 (not: "rfft"
    layers), every decoder linear quantized by quantize_linear with a
    synthetic Hessian and swapped in by replace_with_quantized_linear_.
    Writes tests/golden/ref_ckpt/ (quantized_state.pt, quip_config.json and the
    model's config.json, which the loader uses when the manifest's model id
    cannot be resolved offline) and ref_ckpt_outputs.npz (each quantized
    module's output for a fixed input, and the model's logits, from the
    reference's CPU forward)."""
    sys.path.insert(0, ref_root)
    import torch
    from transformers import AutoModelForCausalLM, LlamaConfig
    from quipsharp.architectures import get_decoder_layers, get_linear_groups
    from quipsharp.checkpoint import build_codebook, replace_with_quantized_linear_, save_quantized_checkpoint
    from quipsharp.quantize import quantize_linear

    torch.set_num_threads(8)
    out_dir = os.path.join(OUT, "ref_ckpt")
    os.makedirs(out_dir, exist_ok=True)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=384, num_hidden_layers=1, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=128, max_position_embeddings=64, attention_bias=True,
                      torch_dtype="float32")
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg).float().eval()
    cb, scale = build_codebook("2bit", "cpu", 0)
    g = torch.Generator().manual_seed(21)
    quantized_modules = []
    for li, layer in enumerate(get_decoder_layers(model)):
        for group in get_linear_groups(layer, li):
            for name, module in group:
                W = module.weight.data.float()
                bias = module.bias.data.float().clone() if module.bias is not None else None
                X = torch.randn(4 * W.shape[1], W.shape[1], generator=g)
                H = X.T @ X / X.shape[0]
                qlayer, _ = quantize_linear(W, H, cb, g=8, damping=1e-2, codebook_scale=scale, tune_iters=2)
                parent_name, _, attr = name.rpartition(".")
                parent = layer.get_submodule(parent_name) if parent_name else layer
                replace_with_quantized_linear_(parent, attr, qlayer, cb, bias=bias)
                quantized_modules.append({"name": f"model.layers.{li}.{name}", "in_features": qlayer.shape[1],
                                          "out_features": qlayer.shape[0],
                                          "transform_kind": "rht" if hasattr(qlayer.signs, "su") else "rfft",
                                          "has_bias": bias is not None})
    save_quantized_checkpoint(model, "tiny-llama-quipsharp", out_dir, bits="2bit", block_size=8, seed=0,
                              quantized_modules=quantized_modules)
    cfg.save_pretrained(out_dir)
    outs = {}
    gx = torch.Generator().manual_seed(22)
    with torch.no_grad():
        for info in quantized_modules:
            mod = model.get_submodule(info["name"])
            x = torch.randn(3, info["in_features"], generator=gx)
            key = info["name"].replace(".", "_")
            outs[key + "_x"] = x.numpy()
            outs[key + "_y"] = mod(x).numpy()
        ids = torch.randint(0, 128, (1, 16), generator=gx)
        outs["ids"] = ids.numpy()
        outs["logits"] = model(ids).logits.float().numpy()
    np.savez_compressed(os.path.join(OUT, "ref_ckpt_outputs.npz"), **outs)
    print("reference checkpoint written to", out_dir, [m["transform_kind"] for m in quantized_modules], flush=True)


if __name__ == "__main__":
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    if len(sys.argv) > 2 and sys.argv[2] == "c1":
        c1_full(root)
    elif len(sys.argv) > 2 and sys.argv[2] == "c1_3bit":
        c1_full_3bit(root)
    elif len(sys.argv) > 2 and sys.argv[2] == "ckpt":
        ref_checkpoint(root)
    else:
        main(root)
