"""Per-configuration measurements at the other model shapes (one MI355X):

* Llama-3-8B layers with 3-bit residual VQ (E8P + E8 1-bit): 4096x4096,
  1024x4096, 14336x4096, 4096x14336.  W ~ N(0, 0.02^2), H = X^T X / 4096 with
  X in R^{4096 x n}; quantize seconds per layer (quantize_linear on the GPU,
  synchronized) and forward time / GB/s at batch 1, 4 and 16.
* Qwen2.5-7B layers with 2-bit E8P: 3584x3584, 512x3584, 18944x3584,
  3584x18944 (3584 = 7 x 512 and 18944 = 37 x 512 take the Kronecker
  transform).  W ~ N(0, 0.02^2) with 1 % of the entries (seeded Bernoulli
  mask) replaced by 0.02 x Student-t(3); quantize seconds per layer and the
  batch-1 forward.
* The Qwen2.5-7B lm_head, 152064 x 3584, left in bf16 as the reference does
  (a dense GEMV through torch), reported separately.

Synthetic seeded data (no checkpoints).  A 512 x 512 quantize runs first, so
that the one-time loading of the solver libraries is not counted in the first
layer.  Forward times: ``reps`` calls of
forward_packed (preallocated workspace and output) captured in one HIP graph,
replayed 5 times, timed with events; GB/s counts the algorithmic bytes (2-byte
E8P codes and 1-byte E8 1-bit codes per 8 weights, bf16 activations in and
out, 1-bit signs, one fp16 scale).  One JSON object on stdout.

    python -m quipsharp_amd.shapes_bench [--tune-iters 10] [--only llama3|qwen25]
"""
import argparse
import json
import sys
import time

import torch

LLAMA3_8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
QWEN25_7B = [(3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)]
QWEN25_VOCAB, QWEN25_HIDDEN = 152064, 3584


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def linear_bytes(m, n, B, stages):
    return m * n // 8 * (2 + (1 if stages == 2 else 0)) + 2 * B * (n + m) + -(-(m + n) // 8) + 2


def make_weights(m, n, heavy, seed):
    """W (m, n) and H = X^T X / 4096 on the CPU, from one seeded generator."""
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(m, n, generator=g) * 0.02
    if heavy:
        mask = torch.rand(m, n, generator=g) < 0.01
        z = torch.randn(m, n, generator=g)
        chi2 = (torch.randn(3, m, n, generator=g) ** 2).sum(0)
        t3 = z / torch.sqrt(chi2 / 3.0)  # Student-t with 3 degrees of freedom
        W = torch.where(mask, 0.02 * t3, W)
    X = torch.randn(4096, n, generator=g)
    return W, X


def time_forward(packed, su, sv, s0, s1, scale, m, n, B, dev, reps=20):
    from quipsharp_amd import _lib
    from quipsharp_amd.quantize import forward_packed
    x = torch.randn(B, n, device=dev).bfloat16()
    ws = torch.zeros(max(_lib.lib().qs_linear_workspace_bytes(m, n, B, packed.layout), 256), dtype=torch.uint8,
                     device=dev)
    out = torch.empty(B, m, dtype=torch.bfloat16, device=dev)
    call = lambda: forward_packed(x, packed, su, sv, s0, s1, scale, out_dtype=torch.bfloat16, workspace=ws, out=out)
    call()
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            call()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (5 * reps)
    del graph
    return us


def quantize_layer(m, n, bits, heavy, seed, tune_iters, dev, codebooks):
    """quantize_linear of one synthetic layer on the GPU: (layer, seconds
    (synchronized), relative proxy loss tr(E H E^T) / tr(W H W^T))."""
    from quipsharp_amd.quantize import quantize_linear
    W, X = make_weights(m, n, heavy, seed)
    Wd, Xd = W.to(dev), X.to(dev)
    H = Xd.T @ Xd / 4096
    del Xd
    cb, scale_in = codebooks[bits]
    torch.manual_seed(seed)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    layer, what_q = quantize_linear(Wd, H, cb, g=8, damping=1e-2, codebook_scale=scale_in, tune_iters=tune_iters)
    torch.cuda.synchronize()
    t_q = time.perf_counter() - t0
    E = layer.signs.reconstruct_weight(what_q) - Wd
    proxy = (torch.trace(E.double() @ H.double() @ E.T.double()) /
             torch.trace(Wd.double() @ H.double() @ Wd.T.double())).item()
    del H, Wd, what_q, E
    return layer, t_q, proxy


def measure_layer(m, n, bits, heavy, seed, batches, tune_iters, dev, codebooks):
    from quipsharp_amd.quantize import PackedCodes, _forward_params
    cb, _ = codebooks[bits]
    layer, t_q, proxy = quantize_layer(m, n, bits, heavy, seed, tune_iters, dev, codebooks)
    stages = layer.codes.shape[0] if layer.codes.dim() == 3 else 1
    kinds, s0, s1 = _forward_params(cb, stages)
    packed = PackedCodes(layer.codes, m, n, kinds)
    su = layer.signs.su.float().contiguous()
    sv = layer.signs.sv.float().contiguous()
    fw = []
    for B in batches:
        us = time_forward(packed, su, sv, s0, s1, layer.scale, m, n, B, dev)
        fw.append({"batch": B, "us": round(us, 2), "GBps": round(linear_bytes(m, n, B, stages) / us / 1e3, 1)})
    rec = {"m": m, "n": n, "stages": stages, "transform": getattr(layer.signs, "kind", "rht"),
           "quantize_s": round(t_q, 3), "relative_proxy_loss": round(proxy, 5), "forward": fw}
    log(json.dumps(rec))
    torch.cuda.empty_cache()
    return rec


def lm_head_gemv(dev, reps=20):
    W = (torch.randn(QWEN25_VOCAB, QWEN25_HIDDEN, device=dev) * 0.02).bfloat16()
    x = torch.randn(1, QWEN25_HIDDEN, device=dev).bfloat16()
    y = x @ W.T
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        torch.matmul(x, W.T, out=y)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    nbytes = W.numel() * 2 + 2 * (QWEN25_HIDDEN + QWEN25_VOCAB)
    return {"m": QWEN25_VOCAB, "n": QWEN25_HIDDEN, "dtype": "bf16", "batch": 1, "us": round(us, 2),
            "GBps": round(nbytes / us / 1e3, 1), "path": "torch.matmul (library GEMV), not quantized"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--tune-iters", type=int, default=10)
    ap.add_argument("--only", choices=["llama3", "qwen25"], default=None)
    args = ap.parse_args()
    from quipsharp_amd.checkpoint import build_codebook
    from quipsharp_amd.quantize import quantize_linear
    dev = torch.device("cuda:0")
    res = {"tune_iters": args.tune_iters, "quantize_timing": "after a 512x512 warm-up quantize (library loading)"}
    # one small layer first: the one-time loading of the solver libraries and
    # kernels stays out of the first measured layer's quantize time
    g = torch.Generator().manual_seed(1)
    W0 = (torch.randn(512, 512, generator=g) * 0.02).to(dev)
    X0 = torch.randn(1024, 512, generator=g).to(dev)
    cb0, s0 = build_codebook("2bit", dev, 0)
    quantize_linear(W0, X0.T @ X0 / 1024, cb0, g=8, damping=1e-2, codebook_scale=s0, tune_iters=1)
    torch.cuda.synchronize()
    if args.only in (None, "llama3"):
        cbs = {"3bit": build_codebook("3bit", dev, 0)}
        res["llama3_8b_rvq3"] = [measure_layer(m, n, "3bit", False, 11 + i, [1, 4, 16], args.tune_iters, dev, cbs)
                                 for i, (m, n) in enumerate(LLAMA3_8B)]
    if args.only in (None, "qwen25"):
        cbs = {"2bit": build_codebook("2bit", dev, 0)}
        res["qwen25_7b_e8p_heavy_tailed"] = [measure_layer(m, n, "2bit", True, 21 + i, [1], args.tune_iters, dev,
                                                           cbs) for i, (m, n) in enumerate(QWEN25_7B)]
        res["qwen25_lm_head_bf16"] = lm_head_gemv(dev)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
