#!/usr/bin/env python3
"""E8P decode-matvec benchmark on one MI355X.

Headline workload (the N=1 line's value, roofline and tok/s): the Qwen3-32B
shape -- 64 decoder layers, each q 8192x5120, k, v 1024x5120, o 5120x8192,
gate, up 25600x5120, down 5120x25600 (m x n), E8P 2-bit random codes (7.8 GB,
30x the Infinity Cache), fp16 per-layer scales, seeded RHT signs (the
non-power-of-two dims take the Kronecker transform: 5120 = 5 x 1024,
25600 = 25 x 1024), bf16 activations, batch 1.  A step is one pass through
the 448 quantized linears in dependency order, q/k/v and gate/up each one
grouped launch (4 launches of linear_fused_kernel per layer), replayed from
a HIP graph: W warm-up replays, then K replays timed with HIP events; value
= algorithmic bytes / step time.  tok_per_s is the greedy decode of the same
model (transformers Qwen3 skeleton, random weights, every decoder linear a
random-code QuantizedLinear): a 512-token random prompt, then 256 new tokens
at batch 1 (and 8), one HIP-graph replay per token.

Also reported, each in its own object: the Qwen3-32B stack at batch 8; the
Llama-2-7B stack (32 layers, 1.62 GB) at batch 1 (grouped and one launch per
linear), 16 (with matrix-core utilisation) and a 512-row prefill; the
Llama-3-8B 3-bit RVQ stack (2.6 GB) at batch 1 / 4 / 16; the Qwen2.5-7B stack
(28 layers, 1.6 GB) at batch 1 with its 152064 x 3584 bf16 lm_head GEMV;
quantize s/layer for the 4096x4096 E8P 2-bit layer and the Llama-3-8B /
Qwen2.5-7B layer shapes; and the reference's CPU path timed on this host
(torch-CPU restatement, oracle/torch_path.py).

Prints one JSON line.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16 matrix-core peak

# Decoder-layer linear stacks: (name, m = out_features, n = in_features) per
# layer, residual-VQ stages (1: E8P 2-bit; 2: E8P + E8 1-bit, 3 bits per
# weight), layer count.
MODELS = {
    "llama2_7b": dict(title="Llama-2-7B", layers=32, stages=1,
                      lin=[("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
                           ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]),
    "llama3_8b": dict(title="Llama-3-8B, 3-bit RVQ (E8P + E8 1-bit)", layers=32, stages=2,
                      lin=[("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                           ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]),
    "qwen25_7b": dict(title="Qwen2.5-7B", layers=28, stages=1,
                      lin=[("q", 3584, 3584), ("k", 512, 3584), ("v", 512, 3584), ("o", 3584, 3584),
                           ("gate", 18944, 3584), ("up", 18944, 3584), ("down", 3584, 18944)]),
    "qwen3_32b": dict(title="Qwen3-32B", layers=64, stages=1,
                      lin=[("q", 8192, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 8192),
                           ("gate", 25600, 5120), ("up", 25600, 5120), ("down", 5120, 25600)]),
}
LLAMA2_7B = MODELS["llama2_7b"]["lin"]
GROUPS = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)]   # linears of one launch, per layer
SOURCE = {"q": None, "k": None, "v": None, "o": "q", "gate": "o", "up": "o", "down": "gate"}
# (m, n) of a Qwen3-32B decoder layer's linears: q, k, v, o, gate, up, down
QWEN3_32B_LINEARS = [(8192, 5120), (1024, 5120), (1024, 5120), (5120, 8192), (25600, 5120), (25600, 5120),
                     (5120, 25600)]


# the distinct layer shapes (m, n) quantized per configuration
LLAMA3_8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
QWEN25_7B = [(3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)]
QWEN25_VOCAB, QWEN25_HIDDEN = 152064, 3584


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--layers", type=int, default=32, help="decoder layers of the Llama-2-7B stack")
    p.add_argument("--skip-quantize", action="store_true")
    p.add_argument("--skip-cpu", action="store_true")
    p.add_argument("--skip-batch16", action="store_true")
    p.add_argument("--skip-alt", action="store_true", help="do not time the other call pattern")
    p.add_argument("--skip-shapes", action="store_true",
                   help="skip the Llama-3-8B and Qwen2.5-7B stacks (and the Qwen2.5-7B lm_head GEMV)")
    p.add_argument("--skip-decode", action="store_true", help="skip the Qwen3-32B-shaped greedy decode")
    p.add_argument("--stack", choices=sorted(STACK_BATCHES), default=None,
                   help="measure only this model's quantized-linear stack and print its record (for profiling)")
    p.add_argument("--stack-batches", default=None,
                   help="comma-separated batch sizes for --stack (default: the ones the full run reports)")
    p.add_argument("--decode-new", type=int, default=256, help="tokens generated per batch size in the decode")
    p.add_argument("--prefill", type=int, default=512,
                   help="rows of the prefill (wide-batch) step also timed; 0 skips it")
    p.add_argument("--per-linear", action="store_true",
                   help="headline with one qs_linear_forward call per linear (the reference's call pattern) "
                        "instead of grouped launches for linears that share an input")
    p.add_argument("--probe", action="store_true",
                   help="hardware-counter probe: one eager step over a 2-layer stack, then a 256 MiB "
                        "elementwise scale (reads and writes 256 MiB) for calibrating byte counters")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def linear_bytes(m, n, B, stages=1):
    """Algorithmic HBM bytes of one quantized-linear call: 2-byte E8P codes
    (plus 1-byte E8 1-bit codes at 3 bits) per 8 weights, bf16 activations in
    and out, 1-bit signs, fp16 scale."""
    return m * n // 8 * (2 + (1 if stages == 2 else 0)) + 2 * B * (n + m) + math.ceil((m + n) / 8) + 2


def mv_bytes(m, n, B, stages=1):
    """Algorithmic bytes of the decode-matvec of one linear.  At B <= 2 that
    is the one-kernel forward (codes, signs, bf16 activations in and out: the
    whole linear); at larger batches the decode-matvec kernel alone (codes,
    fp16 activations in, fp32 partial outputs)."""
    if B <= 2:
        return linear_bytes(m, n, B, stages)
    return m * n // 8 * (2 + (1 if stages == 2 else 0)) + 2 * B * n + 4 * B * m


MV_KERNEL = "linear_fused_kernel"  # the dominant kernel of the batch-1 step
QWEN3_PROFILE = os.path.join(ROOT, "profiles", "linear_fused_qwen3_32b_b1.md")
LLAMA2_PROFILE = os.path.join(ROOT, "profiles", "linear_fused_llama2_7b_b1.md")


def profile_figures(path):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, calibrated) and the
    kernel-only average duration of the batch-1 kernel, from the committed
    rocprofv3 summary of this bench (labelled as such in the output)."""
    out = {}
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    out["traffic"] = int(line.split(":")[1])
                elif line.startswith("kernel_avg_us:"):
                    out["kernel_avg_us"] = float(line.split(":")[1])
    except OSError:
        pass
    return out


class Stack:
    """A synthetic decoder-linear stack (``MODELS`` entry) on the GPU: random
    codes (E8P, plus E8 1-bit for 3-bit layers) packed once, seeded signs."""

    def __init__(self, spec, dev, layers=None):
        import torch
        from quipsharp_amd.hadamard import rademacher
        from quipsharp_amd.quantize import PackedCodes
        self.spec, self.dev = spec, dev
        self.stages = spec["stages"]
        self.shape = {name: (m, n) for name, m, n in spec["lin"]}
        gen = torch.Generator(device=dev).manual_seed(0)
        cpu_gen = torch.Generator().manual_seed(0)
        f16 = lambda v: float(torch.tensor(v, dtype=torch.float16).float())
        self.s0, self.s1 = 1.0, f16(0.47) if self.stages == 2 else 0.0
        # layer scale per linear ~ 0.86 / sqrt(n): each linear keeps the
        # activation norm about level, so a deep stack of random layers stays
        # finite (0.0135 at n = 4096)
        self.scales = {name: f16(0.0135 * math.sqrt(4096 / n)) for name, _, n in spec["lin"]}
        self.layers = []
        for _ in range(layers or spec["layers"]):
            lin = {}
            for name, m, n in spec["lin"]:
                codes = torch.randint(0, 65536, (m, n // 8), generator=gen, device=dev, dtype=torch.int32)
                kinds = [0]
                if self.stages == 2:
                    codes = torch.stack([codes, torch.randint(0, 256, (m, n // 8), generator=gen, device=dev,
                                                              dtype=torch.int32)])
                    kinds = [0, 1]
                packed = PackedCodes(codes, m, n, kinds)
                del codes
                lin[name] = (packed, rademacher(m, device=dev, generator=cpu_gen),
                             rademacher(n, device=dev, generator=cpu_gen))
            self.layers.append(lin)
        torch.cuda.synchronize()

    def code_bytes(self):
        return sum(p[0].nbytes() for lin in self.layers for p in lin.values())


class Runner:
    """Issues one step through the C ABI with preallocated buffers, so it can
    be captured in a HIP graph.  grouped=True runs the linears that share an
    input as one group (qs_linear_forward_group: q/k/v, gate/up; one launch at
    batch 1-2, one launch per stage of the path beyond); otherwise one
    qs_linear_forward per linear (the reference's call pattern)."""

    only = None  # index into plan: steps of that launch only

    def __init__(self, stack, B, grouped=True):
        import ctypes
        import torch
        from quipsharp_amd import _lib
        from quipsharp_amd.hadamard import hartley_matrix, kron_factor
        from quipsharp_amd.quantize import pack_signs
        self.stack, self.B = stack, B
        self.grouped = grouped
        dev = stack.dev
        shape = stack.shape
        self.lib = _lib.lib()
        self._lib = _lib
        g = torch.Generator(device=dev).manual_seed(1)
        n0 = shape["q"][1]
        self.x = torch.randn(B, n0, generator=g, device=dev).bfloat16()
        self.buf = {k: torch.empty(B, m, dtype=torch.bfloat16, device=dev) for k, (m, _) in shape.items()}
        self.K = {}
        for m, n in shape.values():
            for d in (m, n):
                p = kron_factor(d)[0]
                if p > 1 and p not in self.K:
                    self.K[p] = hartley_matrix(p, dev)
        self.plan = GROUPS if self.grouped else [(name,) for name in shape]
        # the grouped entry point takes n a multiple of 256 (one launch at 1-2
        # rows; one launch per stage at 3+ rows up to n = 12288, one forward
        # per linear above)
        self.as_group = [self.grouped and shape[names[0]][1] % 256 == 0 for names in self.plan]
        ws = 0
        for names, grp in zip(self.plan, self.as_group):
            if grp:
                ms = (ctypes.c_int64 * len(names))(*[shape[k][0] for k in names])
                ws = max(ws, self.lib.qs_linear_group_workspace_bytes(shape[names[0]][1], B, len(names), ms))
            else:
                ws = max(ws, self.lib.qs_linear_workspace_bytes(*shape[names[0]], B, _lib.QS_LAYOUT_TILED))
        self.ws = torch.zeros(ws, dtype=torch.uint8, device=dev)  # zero before first use (epoch words)
        # per (layer, launch): the ctypes job array, built once; signs as
        # packed bits (QS_SIGNS_BITS) where the library takes them for this
        # call, as QuantizedLinear passes them
        from quipsharp_amd.quantize import sign_bits_ok
        self.jobs, self._keep = [], []
        for lin in stack.layers:
            per = []
            for names in self.plan:
                arr = (_lib.LinearJob * len(names))()
                src = self.x if SOURCE[names[0]] is None else self.buf[SOURCE[names[0]]]
                bits = all(sign_bits_ok(src, shape[k][0], shape[k][1]) for k in names)
                for j, k in enumerate(names):
                    packed, su, sv = lin[k]
                    if bits:
                        su, sv = pack_signs(su), pack_signs(sv)
                    self._keep += [su, sv]
                    m = shape[k][0]
                    km = kron_factor(m)[0]
                    arr[j] = _lib.LinearJob(packed.codes0.data_ptr(),
                                            None if packed.codes1 is None else packed.codes1.data_ptr(), m,
                                            su.data_ptr(), sv.data_ptr(), km,
                                            self.K[km].data_ptr() if km > 1 else None, stack.s0, stack.s1,
                                            stack.scales[k], None, self.buf[k].data_ptr(), m, 1 if bits else 0)
                per.append(arr)
            self.jobs.append(per)

    def _launch(self, li, gi, names, x, stream):
        from quipsharp_amd.hadamard import kron_factor
        L, _lib = self.lib, self._lib
        n = self.stack.shape[names[0]][1]
        kn = kron_factor(n)[0]
        Kn = self.K[kn].data_ptr() if kn > 1 else None
        if self.as_group[gi]:
            rc = L.qs_linear_forward_group(x.data_ptr(), _lib.QS_DTYPE_BF16, n, self.B, n, kn, Kn, len(names),
                                           self.jobs[li][gi], _lib.QS_DTYPE_BF16, self.ws.data_ptr(), self.ws.numel(),
                                           None, None, stream)
        else:
            assert len(names) == 1, names
            j = self.jobs[li][gi][0]
            layout = _lib.QS_LAYOUT_TILED | (_lib.QS_SIGNS_BITS if j.sign_bits else 0)
            rc = L.qs_linear_forward(
                x.data_ptr(), _lib.QS_DTYPE_BF16, n, self.B, n, j.m, j.codes0, j.codes1, _lib.QS_STAGE_E8_1BIT,
                layout, j.sv, j.su, kn, Kn, j.kron_pm, j.kron_m, j.s0, j.s1, j.layer_scale, None, j.y,
                _lib.QS_DTYPE_BF16, j.m, self.ws.data_ptr(), self.ws.numel(), None, None, stream)
        if rc:
            _lib.check(rc)

    def step(self):
        """One step: every launch of every layer (with ``only`` set, just
        that launch of each layer, reading its usual input buffer)."""
        import torch
        stream = torch.cuda.current_stream(self.stack.dev).cuda_stream
        x = self.x
        for li in range(len(self.stack.layers)):
            for gi, names in enumerate(self.plan):
                if self.only is not None and gi != self.only:
                    continue
                src = x if SOURCE[names[0]] is None else self.buf[SOURCE[names[0]]]
                self._launch(li, gi, names, src, stream)
            if self.only is None:
                x = self.buf["down"]
        return self.out()

    def out(self):
        return self.buf["down" if self.only is None else self.plan[self.only][-1]]

    def launches_per_step(self):
        return len(self.stack.layers) * (len(self.plan) if self.only is None else 1)

    def bytes_per_step(self):
        st = self.stack.stages
        return len(self.stack.layers) * sum(linear_bytes(m, n, self.B, st) for m, n in self.stack.shape.values())

    def mv_bytes_per_step(self):
        """Algorithmic bytes of the step's decode-matvec launches (at 1-2 rows
        a grouped launch reads its shared input once)."""
        st, shape, B = self.stack.stages, self.stack.shape, self.B
        if B <= 2:
            per = 0
            for names in self.plan:
                n = shape[names[0]][1]
                per += sum(linear_bytes(*shape[k], B, st) for k in names) - (len(names) - 1) * 2 * B * n
            return len(self.stack.layers) * per
        return len(self.stack.layers) * sum(mv_bytes(m, n, B, st) for m, n in shape.values())


def time_graph(runner, steps, warmup):
    """Captures one step in a HIP graph (checked against the eager step),
    replays it ``warmup`` times, then times ``steps`` replays back to back
    with a HIP event after each: returns the mean (the whole timed region
    over ``steps``) and the median replay, in ms."""
    import torch
    dev = runner.stack.dev
    ref = runner.step().clone()
    torch.cuda.synchronize()
    if not torch.isfinite(ref).all():
        raise RuntimeError("the stack's outputs are not finite")
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        runner.step()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        runner.step()
    for _ in range(max(warmup, 1)):
        graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(runner.out(), ref):
        raise RuntimeError("graph replay differs from the eager step")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(steps):
        graph.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    if not torch.equal(runner.out(), ref):
        raise RuntimeError("graph replays are not reproducible")
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    del graph
    return {"mean_ms": ev[0].elapsed_time(ev[steps]) / steps, "median_ms": statistics.median(per),
            "min_ms": min(per), "max_ms": max(per)}


def time_eager(runner, steps, warmup):
    """ms per step, issued eagerly (the wide-batch path calls a library GEMM,
    which is not captured in a graph)."""
    import torch
    for _ in range(max(warmup, 1)):
        runner.step()
    torch.cuda.synchronize()
    ref = runner.buf["down"].clone()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        runner.step()
    e1.record()
    torch.cuda.synchronize()
    if not torch.equal(runner.buf["down"], ref):
        raise RuntimeError("prefill steps are not reproducible")
    return e0.elapsed_time(e1) / steps


def gpu_quantize(dev, n=4096, tune_iters=10):
    import torch
    from quipsharp_amd.checkpoint import build_codebook
    from quipsharp_amd.quantize import quantize_linear, linear_forward
    g = torch.Generator().manual_seed(0)
    W = torch.randn(n, n, generator=g) * 0.02
    X = torch.randn(2048, n, generator=g)
    x = torch.randn(n, generator=g)
    Wd, Xd = W.to(dev), X.to(dev)
    H = Xd.T @ Xd / 2048
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    cb, s = build_codebook("2bit", dev, 0)
    torch.cuda.synchronize()
    t_cb = time.perf_counter() - t0
    # one other layer of the same shape first (one refinement iteration): the
    # one-time loading of the solver libraries and the library GEMMs' kernel
    # selection for these shapes stay out of the per-layer time, as in a
    # model's run, where every layer shape repeats across the layers
    gw = torch.Generator().manual_seed(1)
    W0 = (torch.randn(n, n, generator=gw) * 0.02).to(dev)
    X0 = torch.randn(1024, n, generator=gw).to(dev)
    quantize_linear(W0, X0.T @ X0 / 1024, cb, g=8, damping=1e-2, codebook_scale=s, tune_iters=1)
    torch.manual_seed(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    layer, what_q = quantize_linear(Wd, H, cb, g=8, damping=1e-2, codebook_scale=s, tune_iters=tune_iters)
    torch.cuda.synchronize()
    t_q = time.perf_counter() - t0
    y = linear_forward(x.to(dev), layer, cb)
    W_q = layer.signs.reconstruct_weight(what_q)
    E = W_q - Wd
    proxy = torch.trace(E.double() @ H.double() @ E.T.double()).item() / torch.trace(
        Wd.double() @ H.double() @ Wd.T.double()).item()
    return {"quantize_s_per_layer": round(t_q, 4),
            "timing": "after a warm-up quantize of another layer of the same shape (library loading and kernel "
                      "selection), as for the second and later layers of a model",
            "codebook_fit_s": round(t_cb, 4), "codebook_scale": s,
            "relative_proxy_loss": round(proxy, 5), "forward_ok": bool(torch.isfinite(y).all().item())}


def cpu_baseline(dev_layers_sample=1):
    """The reference's CPU path (torch-CPU restatement) on this host:
    forward for one decoder layer's 7 linears at batch 1 (dense dequantize
    loop + matmul; RHT for power-of-two dims, RFFT for 11008), and a timed
    sample of the 4096x4096 quantize extrapolated to the full layer."""
    import torch
    from oracle import torch_path
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    # forward, one decoder layer
    t_fwd = 0.0
    nbytes = 0
    for name, m, n in LLAMA2_7B:
        codes = torch.randint(0, 65536, (m, n // 8), generator=g)
        x = torch.randn(1, n, generator=g)
        kw = {}
        if m == 4096 and n == 4096:
            kw = dict(su=torch.randint(0, 2, (m,), generator=g).float() * 2 - 1,
                      sv=torch.randint(0, 2, (n,), generator=g).float() * 2 - 1)
        else:
            ph = lambda k: torch.polar(torch.ones(k), torch.rand(k, generator=g) * 2 * math.pi)
            kw = dict(phase_u=ph(m // 2), phase_v=ph(n // 2))
        t0 = time.perf_counter()
        torch_path.linear_forward(x, codes, 0.0135, **kw)
        t_fwd += time.perf_counter() - t0
        nbytes += linear_bytes(m, n, 1)
    # quantize sample at 4096 x 4096
    W = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(0)) * 0.02
    X = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(1))
    H = X.T @ X / 2048
    H = H + 1e-2 * H.diagonal().mean() * torch.eye(4096)
    su = torch.randint(0, 2, (4096,), generator=g).float() * 2 - 1
    sv = torch.randint(0, 2, (4096,), generator=g).float() * 2 - 1
    t0 = time.perf_counter()
    what = torch_path.fwht(torch_path.fwht(W * su[:, None] * sv[None, :], 0), 1)
    hhat = torch_path.fwht(torch_path.fwht(H * sv[:, None] * sv[None, :], 0), 1)
    L = torch_path.block_ldl(hhat, 8)
    what = what / (what.pow(2).mean().sqrt().item() * 0.95)
    t_setup = time.perf_counter() - t0
    T = 512
    base_k = [T - 1, 3 * T // 4, T // 2, T // 4, 0]
    t0 = time.perf_counter()
    torch_path.quantize_steps(what, L, hhat, base_k)
    t_base = (time.perf_counter() - t0) / len(base_k)
    tune_k = [T - 1, T // 2, 0]
    t0 = time.perf_counter()
    torch_path.quantize_steps(what, L, hhat, tune_k, tune=True)
    t_tune = (time.perf_counter() - t0) / len(tune_k)
    q_total = t_setup + T * t_base + 10 * T * t_tune
    # Qwen3-32B-shaped decode: one decoder layer's 7 linears at batch 1 (RHT
    # where both dims are powers of two, RFFT otherwise, as the reference
    # chooses), times 64 layers
    t_q3 = 0.0
    for m, n in QWEN3_32B_LINEARS:
        codes = torch.randint(0, 65536, (m, n // 8), generator=g)
        x = torch.randn(1, n, generator=g)
        if m & (m - 1) == 0 and n & (n - 1) == 0:
            kw = dict(su=torch.randint(0, 2, (m,), generator=g).float() * 2 - 1,
                      sv=torch.randint(0, 2, (n,), generator=g).float() * 2 - 1)
        else:
            ph = lambda k: torch.polar(torch.ones(k), torch.rand(k, generator=g) * 2 * math.pi)
            kw = dict(phase_u=ph(m // 2), phase_v=ph(n // 2))
        t0 = time.perf_counter()
        torch_path.linear_forward(x, codes, 0.0135, **kw)
        t_q3 += time.perf_counter() - t0
        del codes
    q3_bytes = sum(linear_bytes(m, n, 1) for m, n in QWEN3_32B_LINEARS)
    return {
        "qwen3_32b_decode_s_per_token_extrapolated": 64 * t_q3, "qwen3_32b_GBps": q3_bytes / t_q3 / 1e9,
        "forward_GBps": nbytes / t_fwd / 1e9, "forward_s_per_decoder_layer": t_fwd,
        "quantize_s_per_layer_extrapolated": q_total, "quantize_step_s": {"base": t_base, "tune": t_tune},
        "threads": threads, "host": host_cpu(),
    }


def host_cpu():
    """Model, sockets and physical cores of this host, from /proc/cpuinfo."""
    model, cores = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            phys = core = None
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
            if phys is not None:
                cores.add((phys, core))
    except OSError:
        pass
    return {"model": model, "sockets": len({p for p, _ in cores}) or None, "physical_cores": len(cores) or None,
            "threads_available": os.cpu_count()}


def hbm_copy_peak(dev, nbytes=1 << 30, reps=10):
    """Measured device-to-device copy rate (bytes read + written per second)
    over a 1 GiB buffer: the practical HBM ceiling beside the 8 TB/s peak."""
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).uniform_()
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    gbps = 2 * nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return round(gbps, 1)


def kernel_rates(dev):
    """Throughput of the quantize-time kernels: E8P nearest-codeword encode
    (8-weight groups per second) and the RHT along rows and columns of a
    4096 x 4096 fp32 matrix (8 bytes per element per pass)."""
    import torch
    from quipsharp_amd.codebooks.e8p import E8PCodebook
    from quipsharp_amd.hadamard import fwht
    g = torch.Generator(device=dev).manual_seed(3)
    cb = E8PCodebook(device=dev)
    ngroups = 1 << 21
    x = torch.randn(ngroups, 8, generator=g, device=dev)
    W = torch.randn(4096, 4096, generator=g, device=dev)
    out = {}
    for name, fn, reps in (("encode", lambda: cb.quantize(x), 5), ("fwht_rows", lambda: fwht(W, 1), 20),
                           ("fwht_cols", lambda: fwht(W, 0), 20)):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) * 1e-3 / reps
    return {"e8p_encode_groups_per_s": round(ngroups / out["encode"], 0), "e8p_encode_groups": ngroups,
            "fwht_4096x4096_rows_GBps": round(8 * W.numel() / out["fwht_rows"] / 1e9, 1),
            "fwht_4096x4096_cols_GBps": round(8 * W.numel() / out["fwht_cols"] / 1e9, 1)}


# batch sizes each layer stack is measured at
STACK_BATCHES = {"llama2_7b": [1, 16], "llama3_8b": [1, 4, 16], "qwen25_7b": [1], "qwen3_32b": [1, 8]}


def stack_batches(key, batches, steps, warmup, dev):
    """ms/step, GB/s and tok/s of a ``MODELS`` stack at each batch size
    (grouped launches, graph-replayed steps)."""
    import torch
    spec = MODELS[key]
    t0 = time.perf_counter()
    stack = Stack(spec, dev)
    out = {"workload": f"{spec['title']} quantized-linear stack, {spec['layers']} decoder layers",
           "linears": {name: [m, n] for name, m, n in spec["lin"]}, "bits": 3 if spec["stages"] == 2 else 2,
           "code_bytes": stack.code_bytes(), "setup_s": round(time.perf_counter() - t0, 1), "batches": []}
    for B in batches:
        r = Runner(stack, B)
        t = time_graph(r, steps, warmup)
        ms = t["mean_ms"]
        rec = {"batch": B, "ms_per_step": round(ms, 4), "median_ms_per_step": round(t["median_ms"], 4),
               "GBps": round(r.bytes_per_step() / ms / 1e6, 1), "tok_per_s": round(B * 1e3 / ms, 1),
               "launches_per_step": r.launches_per_step()}
        if B <= 2:
            rec["launches"] = launch_rates(r, steps, warmup)
        out["batches"].append(rec)
        log(f"{key} batch {B}: {ms:.3f} ms/step, {r.bytes_per_step() / ms / 1e6:.1f} GB/s"
            + "".join(f"; {l['launch']} {l['us_per_launch']} us {l['GBps']} GB/s" for l in rec.get("launches", [])))
        del r
    del stack
    torch.cuda.empty_cache()
    return out


def launch_rates(runner, steps, warmup):
    """Per launch of each group (q+k+v, o, gate+up, down), timed alone over
    every layer of the stack (graph replays, codes rotated through HBM): us
    per launch and algorithmic GB/s."""
    out = []
    stack, B = runner.stack, runner.B
    for gi, names in enumerate(runner.plan):
        runner.only = gi
        t = time_graph(runner, steps, warmup)
        us = t["mean_ms"] * 1e3 / len(stack.layers)
        nbytes = sum(linear_bytes(*stack.shape[k], B, stack.stages) for k in names)
        out.append({"launch": "+".join(names), "shapes": [list(stack.shape[k]) for k in names],
                    "us_per_launch": round(us, 2), "median_us_per_launch": round(t["median_ms"] * 1e3 / len(stack.layers), 2),
                    "GBps": round(nbytes / us / 1e3, 1)})
    runner.only = None
    return out


def make_weights(m, n, heavy, seed):
    """W (m, n) ~ 0.02 N(0, 1) and calibration rows X (4096, n) ~ N(0, 1) on
    the CPU from one seeded generator; heavy: 1 % of the entries of W (seeded
    Bernoulli mask) replaced by 0.02 x Student-t(3)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(m, n, generator=g) * 0.02
    if heavy:
        mask = torch.rand(m, n, generator=g) < 0.01
        z = torch.randn(m, n, generator=g)
        chi2 = (torch.randn(3, m, n, generator=g) ** 2).sum(0)
        W = torch.where(mask, 0.02 * z / torch.sqrt(chi2 / 3.0), W)
    X = torch.randn(4096, n, generator=g)
    return W, X


def quantize_layer(m, n, bits, heavy, seed, tune_iters, dev, codebooks):
    """quantize_linear of one synthetic layer on the GPU (H = X^T X / 4096):
    (layer, seconds (synchronized), relative proxy loss tr(E H E^T) / tr(W H W^T))."""
    import torch
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


def shape_quantize(dev, tune_iters=10):
    """Quantize s/layer at the Llama-3-8B (3-bit RVQ) and Qwen2.5-7B (2-bit,
    1 % Student-t(3) outliers) layer shapes."""
    from quipsharp_amd.checkpoint import build_codebook
    out = {}
    for key, shapes, bits, heavy, seed in (("llama3_8b_3bit", LLAMA3_8B, "3bit", False, 11),
                                          ("qwen25_7b_2bit_heavy_tailed", QWEN25_7B, "2bit", True, 21)):
        cbs = {bits: build_codebook(bits, dev, 0)}
        rows = []
        for i, (m, n) in enumerate(shapes):
            _, t_q, proxy = quantize_layer(m, n, bits, heavy, seed + i, tune_iters, dev, cbs)
            rows.append({"m": m, "n": n, "quantize_s": round(t_q, 3), "relative_proxy_loss": round(proxy, 5)})
            log(f"quantize {key} {m}x{n}: {t_q:.3f} s")
        out[key] = rows
    return out


def lm_head_gemv(dev, reps=20):
    """The Qwen2.5-7B lm_head (152064 x 3584), left in bf16 as the reference
    leaves it (only decoder linears are quantized): one library GEMV through
    torch at batch 1, us and GB/s (weights + activations)."""
    import torch
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
    del W
    torch.cuda.empty_cache()
    return {"m": QWEN25_VOCAB, "n": QWEN25_HIDDEN, "dtype": "bf16", "batch": 1, "us": round(us, 2),
            "GBps": round(nbytes / us / 1e3, 1), "path": "torch.matmul (library GEMV), not quantized"}


def llama2_7b_records(dev, args):
    """The Llama-2-7B stack: batch 1 (grouped and one launch per linear,
    per-launch rates), 16 rows (with matrix-core utilisation) and a prefill."""
    import torch
    spec = MODELS["llama2_7b"]
    t_setup = time.perf_counter()
    stack = Stack(spec, dev, args.layers)
    log(f"llama2_7b stack: {args.layers} layers, {stack.code_bytes() / 1e9:.2f} GB of codes, "
        f"setup {time.perf_counter() - t_setup:.1f}s")
    out = {"workload": "Llama-2-7B quantized-linear stack (q,k,v,o 4096x4096; gate,up 11008x4096; down "
                       "4096x11008) x %d decoder layers, E8P 2-bit random codes" % args.layers,
           "code_bytes": stack.code_bytes()}
    r1 = Runner(stack, 1, grouped=not args.per_linear)
    t1 = time_graph(r1, args.steps, args.warmup)
    ms = t1["mean_ms"]
    launches = r1.launches_per_step()
    mv_ms = ms / launches
    achieved = r1.mv_bytes_per_step() / launches / (mv_ms * 1e-3) / 1e9
    prof = profile_figures(LLAMA2_PROFILE)
    out["batch1"] = {"ms_per_step": round(ms, 4), "median_ms_per_step": round(t1["median_ms"], 4),
                     "GBps": round(r1.bytes_per_step() / ms / 1e6, 1),
                     "linear_stack_steps_per_s": round(1e3 / ms, 1), "launches_per_step": launches,
                     "call_pattern": "grouped" if r1.grouped else "per-linear",
                     "roofline": {"kernel": MV_KERNEL, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                                  "avg_launch_us": round(mv_ms * 1e3, 3),
                                  "bytes_per_launch": int(r1.mv_bytes_per_step() / launches),
                                  "profile_kernel_avg_us": prof.get("kernel_avg_us"),
                                  "traffic": prof.get("traffic") if args.layers == 32 and r1.grouped else None}}
    log(f"llama2_7b batch 1: {ms:.3f} ms/step, {out['batch1']['GBps']} GB/s")
    if r1.grouped:
        out["batch1"]["launches"] = launch_rates(r1, args.steps, args.warmup)
    if not args.skip_alt:
        r_alt = Runner(stack, 1, grouped=args.per_linear)
        ta = time_graph(r_alt, args.steps, args.warmup)
        out["batch1_" + ("grouped" if r_alt.grouped else "per_linear")] = {
            "ms_per_step": round(ta["mean_ms"], 4), "median_ms_per_step": round(ta["median_ms"], 4),
            "GBps": round(r1.bytes_per_step() / ta["mean_ms"] / 1e6, 1),
            "launches_per_step": r_alt.launches_per_step()}
        del r_alt
    if not args.skip_batch16:
        r16 = Runner(stack, 16, grouped=not args.per_linear)
        t16 = time_graph(r16, args.steps, args.warmup)
        ms16 = t16["mean_ms"]
        flops = 2 * 16 * args.layers * sum(m * n for _, m, n in LLAMA2_7B)
        tf = flops / ms16 / 1e9
        out["batch16"] = {"ms_per_step": round(ms16, 4), "median_ms_per_step": round(t16["median_ms"], 4),
                          "GBps": round(r16.bytes_per_step() / ms16 / 1e6, 1),
                          "tok_per_s": round(16 * 1e3 / ms16, 1), "TFLOPs": round(tf, 2),
                          "mfma_frac_fp16_dense": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                          "call_pattern": "grouped" if r16.grouped else "per-linear",
                          "launches_per_step": r16.launches_per_step()}
        log(f"llama2_7b batch 16: {ms16:.3f} ms/step")
        del r16
    if args.prefill > 0:
        P = args.prefill
        rp = Runner(stack, P, grouped=not args.per_linear)
        msp = time_eager(rp, max(args.steps // 10, 3), 2)
        flops = 2 * P * args.layers * sum(m * n for _, m, n in LLAMA2_7B)
        out["prefill"] = {"rows": P, "ms_per_step": round(msp, 3), "tok_per_s": round(P * 1e3 / msp, 1),
                          "TFLOPs": round(flops / msp / 1e9, 1),
                          "mfma_frac_fp16_dense": round(flops / msp / 1e9 / MFMA_F16_PEAK_TFLOPS, 4),
                          "call_pattern": "grouped" if rp.grouped else "per-linear",
                          "path": "wp_kernel: 4 waves decode E8P codes (with their +-1/4 shifts) into fp16 "
                                  "32x32x16 MFMA fragments in LDS, 4 waves multiply them (fp32 accumulate)"}
        log(f"llama2_7b prefill {P} rows: {msp:.3f} ms/step")
        del rp
    del stack
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs its kernels on a single MI355X "
              f"(no multi-GPU path); got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    if args.stack:
        batches = ([int(b) for b in args.stack_batches.split(",")] if args.stack_batches
                   else STACK_BATCHES[args.stack])
        print(json.dumps({"stack": args.stack, **stack_batches(args.stack, batches, args.steps, args.warmup, dev)}))
        return
    if args.probe:
        stack = Stack(MODELS["llama2_7b"], dev, 2)
        r1 = Runner(stack, 1)
        r1.step()
        torch.cuda.synchronize()
        Runner(stack, 16).step()           # batch-16 matvec
        torch.cuda.synchronize()
        Runner(stack, 512).step()          # prefill (wide GEMM)
        torch.cuda.synchronize()
        gpu_quantize(dev, n=1024, tune_iters=1)  # encode / LDLQ kernels
        torch.cuda.synchronize()
        from quipsharp_amd.codebooks.e8p import E8PCodebook
        E8PCodebook(device=dev).quantize(torch.randn(1 << 20, 8, device=dev))  # one large encode
        torch.cuda.synchronize()
        a = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        torch.mul(a, 2.0, out=b)
        torch.cuda.synchronize()
        print(json.dumps({"probe": "done", "linears": r1.launches_per_step(), "copy_bytes": a.numel() * 4}))
        return
    # headline: the Qwen3-32B stack at batch 1 (and 8)
    spec = MODELS["qwen3_32b"]
    t_setup = time.perf_counter()
    stack = Stack(spec, dev)
    log(f"qwen3_32b stack: {len(stack.layers)} layers, {stack.code_bytes() / 1e9:.2f} GB of codes, "
        f"setup {time.perf_counter() - t_setup:.1f}s")
    r1 = Runner(stack, 1)
    t1 = time_graph(r1, args.steps, args.warmup)
    ms = t1["mean_ms"]
    bps = r1.bytes_per_step()
    value = bps / (ms * 1e-3) / 1e9
    launches = r1.launches_per_step()
    # every launch of the batch-1 step is the dominant kernel: its average
    # launch duration over the timed region is the step over the launches
    # (the gaps between the dependent launches included)
    mv_ms = ms / launches
    mv_avg_bytes = r1.mv_bytes_per_step() / launches
    achieved = mv_avg_bytes / (mv_ms * 1e-3) / 1e9
    log(f"qwen3_32b batch 1: {ms:.3f} ms/step (median {t1['median_ms']:.3f}), {value:.1f} GB/s, "
        f"{mv_ms * 1e3:.2f} us per launch -> {achieved:.1f} GB/s")
    extra = {"qwen3_32b_stack": {"workload": spec["title"] + " quantized-linear stack, 64 decoder layers",
                                 "batch1_launches": launch_rates(r1, args.steps, args.warmup)}}
    log("launches: " + "; ".join(f"{l['launch']} {l['us_per_launch']} us {l['GBps']} GB/s"
                                 for l in extra["qwen3_32b_stack"]["batch1_launches"]))
    del r1
    for B in STACK_BATCHES["qwen3_32b"][1:]:
        rb = Runner(stack, B)
        tb = time_graph(rb, args.steps, args.warmup)
        extra["qwen3_32b_stack"][f"batch{B}"] = {
            "ms_per_step": round(tb["mean_ms"], 4), "median_ms_per_step": round(tb["median_ms"], 4),
            "GBps": round(rb.bytes_per_step() / tb["mean_ms"] / 1e6, 1), "launches_per_step": rb.launches_per_step()}
        log(f"qwen3_32b batch {B}: {tb['mean_ms']:.3f} ms/step")
        del rb
    code_bytes = stack.code_bytes()
    del stack
    torch.cuda.empty_cache()
    decode = None
    if not args.skip_decode:
        from quipsharp_amd.decode import measure_decode
        decode = measure_decode(new=args.decode_new, device=str(dev))
        extra["qwen3_32b_decode"] = decode
        for run in decode["runs"]:
            log(f"qwen3-32b decode batch {run['batch']}: {run['tok_per_s']} tok/s, {run['ms_per_step']} ms/step "
                f"({run['linears_ms_per_step']} ms in the quantized linears)")
    extra["llama2_7b_stack"] = llama2_7b_records(dev, args)
    if not args.skip_shapes:
        extra["llama3_8b_3bit_stack"] = stack_batches("llama3_8b", STACK_BATCHES["llama3_8b"], args.steps,
                                                      args.warmup, dev)
        extra["qwen25_7b_stack"] = stack_batches("qwen25_7b", STACK_BATCHES["qwen25_7b"], args.steps, args.warmup, dev)
        extra["qwen25_7b_lm_head_bf16"] = lm_head_gemv(dev)
        log(f"qwen2.5-7b lm_head (bf16 GEMV): {extra['qwen25_7b_lm_head_bf16']}")
    if not args.skip_quantize:
        extra["quantize_4096x4096_e8p_2bit"] = gpu_quantize(dev)
        log(f"quantize: {extra['quantize_4096x4096_e8p_2bit']}")
        extra["quantize_layer_shapes"] = shape_quantize(dev)
        extra["quantize_kernels"] = kernel_rates(dev)
        log(f"quantize kernels: {extra['quantize_kernels']}")
    copy_peak = hbm_copy_peak(dev)
    log(f"measured copy rate: {copy_peak} GB/s")
    cpu = None
    if not args.skip_cpu:
        log("timing the reference CPU path ...")
        c = cpu_baseline()
        cpu = {"value": round(c["qwen3_32b_decode_s_per_token_extrapolated"], 1), "unit": "s/token",
               "cores": c["threads"], "kind": "port", "host": c["host"],
               "sample": "reference forward (dense dequantize loop + fp32 matmul; RHT where both dims are powers "
                         "of two, RFFT otherwise, as the reference chooses) of one Qwen3-32B decoder layer's 7 "
                         "linears at batch 1, torch-CPU restatement, x 64 layers = s per token of the decoder "
                         "linears",
               "qwen3_32b_GBps": round(c["qwen3_32b_GBps"], 3),
               "llama2_7b_forward_GBps": round(c["forward_GBps"], 3),
               "llama2_7b_forward_s_per_decoder_layer": round(c["forward_s_per_decoder_layer"], 3),
               "quantize_s_per_layer": round(c["quantize_s_per_layer_extrapolated"], 1),
               "quantize_sample": "4096x4096 E8P 2-bit, extrapolated from 5 base-pass and 3 refinement steps"}
        if "quantize_4096x4096_e8p_2bit" in extra:
            extra["quantize_speedup_vs_cpu"] = round(
                c["quantize_s_per_layer_extrapolated"] / extra["quantize_4096x4096_e8p_2bit"]["quantize_s_per_layer"], 1)
    prof = profile_figures(QWEN3_PROFILE)
    runs = {r["batch"]: r for r in decode["runs"]} if decode else {}
    line = {
        "metric": "E8P decode-matvec HBM GB/s (% peak) + batch-1 tok/s; quantize s/layer",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "median_ms_per_step": round(t1["median_ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "e8p-2bit codes, fp16 x fp16 -> fp32 accumulate (bf16 in/out)", "data": "synthetic",
        "config": {"workload": "Qwen3-32B quantized-linear stack: 64 decoder layers x (q 8192x5120; k, v "
                               "1024x5120; o 5120x8192; gate, up 25600x5120; down 5120x25600), E8P 2-bit random "
                               "codes, batch 1",
                   "global_batch": 1, "layers": 64, "linears_per_step": 7 * 64, "launches_per_step": launches,
                   "call_pattern": "grouped (q/k/v and gate/up share a launch)", "code_bytes": code_bytes,
                   "parallelism": "none (1 GPU)"},
        "tok_per_s": runs[1]["tok_per_s"] if 1 in runs else None,
        "tok_per_s_source": "greedy decode of the Qwen3-32B-shaped model (512-token prompt, %d new tokens), "
                            "batch 1, one HIP-graph replay per token" % args.decode_new,
        "tok_per_s_batch8": runs[8]["tok_per_s"] if 8 in runs else None,
        "linear_stack_steps_per_s": round(1e3 / ms, 1),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "kernel": MV_KERNEL, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(mv_ms * 1e3, 3), "bytes_per_launch": int(mv_avg_bytes),
                     "launch_time_source": "timed graph replays: step time / launches (the gaps between the "
                                           "dependent launches included)",
                     "profile_kernel_avg_us": prof.get("kernel_avg_us"),
                     "measured_copy_GBps": copy_peak,
                     "frac_of_measured_copy": round(achieved / copy_peak, 4) if copy_peak else None,
                     "traffic": prof.get("traffic"),
                     "traffic_source": "committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary "
                                       "(profiles/linear_fused_qwen3_32b_b1.md), not measured in this run"},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
