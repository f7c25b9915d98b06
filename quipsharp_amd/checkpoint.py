"""Codebook construction, the quantized ``nn.Module`` and the compact
checkpoint format (quipsharp/checkpoint.py).

``QuantizedLinear`` keeps the reference's buffers (int16 ``codes``, fp32
``scale``, ``su``/``sv`` signs or ``phase_u``/``phase_v`` RFFT phases,
optional ``bias``) so state dicts move between the two implementations; on
first use on a device the codes are repacked once into the kernel layout (a
non-persistent cache), and ``forward`` runs the fused decode + transform +
matvec kernels in the activation dtype (bf16/fp16/fp32) without a dense
weight.  ``save_quantized_checkpoint`` / ``load_quantized_checkpoint`` read
and write the reference's format (state dict + manifest).
"""
import ctypes
import json
import warnings
import weakref
from pathlib import Path

import torch
from torch import nn, Tensor

from .codebooks.e8_1bit import E8OneBitCodebook
from .codebooks.e8p import E8PCodebook
from .incoherence import IncoherenceSigns, KronSigns
from .quantize import (PackedCodes, QuantizedLayer, RVQCodebookAdapter, _forward_params, decode_matvec,
                       forward_packed)
from .rfft import RFFTPhases
from .rvq import RVQStage, fit_residual_stage_scale, fit_stage_scale


def num_rvq_stages(bits: str) -> int:
    """quipsharp/checkpoint.py:56-57."""
    return 1 if bits == "2bit" else 2


def build_codebook(bits: str, device, seed: int = 0):
    """(codebook, fitted input scale) for "2bit" (E8P), "3bit" (E8P + E8 1-bit)
    or "4bit" (E8P + E8P) -- quipsharp/checkpoint.py:60-77, same seeds and
    sample counts, so the same scales are chosen."""
    e8p = E8PCodebook(device=device)
    e8p_scale = fit_stage_scale(e8p, seed=seed, device=device, n_samples=20_000)
    if bits == "2bit":
        return e8p, e8p_scale
    second = E8OneBitCodebook(device=device) if bits == "3bit" else E8PCodebook(device=device)
    second_scale = fit_residual_stage_scale([RVQStage(e8p, e8p_scale)], second, seed=seed + 1, device=device,
                                            n_samples=20_000)
    rvq_cb = RVQCodebookAdapter([RVQStage(e8p, e8p_scale), RVQStage(second, second_scale)])
    rvq_scale = fit_stage_scale(rvq_cb, seed=seed + 2, device=device, n_samples=20_000)
    return rvq_cb, rvq_scale


class QuantizedLinear(nn.Module):
    """Drop-in for a quantized nn.Linear (quipsharp/checkpoint.py:80-146).

    transform_kind: "rht" (power-of-two dims), "krht" (Kronecker transform,
    this library's choice for other dims) or "rfft" (the reference's choice
    for other dims: complex64 ``phase_u``/``phase_v`` buffers, FFTs in hipFFT
    around the library's decode-matvec).
    """

    def __init__(self, in_features: int, out_features: int, g: int, transform_kind: str, num_stages: int = 1,
                 has_bias: bool = False):
        super().__init__()
        if transform_kind not in ("rht", "krht", "rfft"):
            raise NotImplementedError(f"transform_kind {transform_kind!r} is not supported (rht, krht, rfft)")
        self.in_features = in_features
        self.out_features = out_features
        self.g = g
        self.transform_kind = transform_kind
        self.num_stages = num_stages
        self.codebook = None  # assigned by the caller
        self.register_buffer("bias", torch.zeros(out_features) if has_bias else None)
        T = in_features // g
        shape = (out_features, T) if num_stages == 1 else (num_stages, out_features, T)
        self.register_buffer("codes", torch.zeros(shape, dtype=torch.int16))
        self.register_buffer("scale", torch.zeros(()))
        if transform_kind == "rfft":
            self.register_buffer("phase_u", torch.zeros(out_features // 2, dtype=torch.complex64))
            self.register_buffer("phase_v", torch.zeros(in_features // 2, dtype=torch.complex64))
        else:
            self.register_buffer("su", torch.zeros(out_features))
            self.register_buffer("sv", torch.zeros(in_features))
        self._packed = None
        self._packed_key = None
        self._ws = None  # forward workspace (zeroed once; reused, so the forward can be graph-captured)
        self._siblings = None  # linked linears that read the same input (link_sibling_linears)
        self._sib_out = None   # (weakref to x, x._version, output) left by a sibling's grouped forward

    @classmethod
    def from_quantized_layer(cls, layer: QuantizedLayer, bias: Tensor = None) -> "QuantizedLinear":
        m, n = layer.shape
        kind = getattr(layer.signs, "kind", None)
        if kind not in ("rht", "krht", "rfft"):
            raise NotImplementedError("only Hadamard, Kronecker and RFFT-transformed layers are supported")
        stages = layer.codes.shape[0] if layer.codes.dim() == 3 else 1
        mod = cls(in_features=n, out_features=m, g=layer.g, transform_kind=kind, num_stages=stages,
                  has_bias=bias is not None)
        with torch.no_grad():
            mod.codes.copy_(layer.codes)
            mod.scale.copy_(torch.as_tensor(layer.scale, dtype=torch.float32))
            if bias is not None:
                mod.bias.copy_(bias.float())
            if kind == "rfft":
                mod.phase_u.copy_(layer.signs.phase_u)
                mod.phase_v.copy_(layer.signs.phase_v)
            else:
                mod.su.copy_(layer.signs.su)
                mod.sv.copy_(layer.signs.sv)
        return mod

    def _quantized_layer(self) -> QuantizedLayer:
        codes = self.codes.to(torch.int64) & 0xFFFF
        if self.transform_kind == "rfft":
            signs = RFFTPhases(phase_u=self.phase_u, phase_v=self.phase_v)
        else:
            cls = IncoherenceSigns if self.transform_kind == "rht" else KronSigns
            signs = cls(su=self.su, sv=self.sv)
        return QuantizedLayer(codes=codes, signs=signs, g=self.g, shape=(self.out_features, self.in_features),
                              scale=self.scale.item())

    def _load_from_state_dict(self, *args, **kwargs):
        self._packed = None
        self._bits_key = None
        self._f32_cache = {}
        self._sib_out = None
        return super()._load_from_state_dict(*args, **kwargs)

    def _apply(self, fn, *args, **kwargs):
        self._packed = None
        self._bits_key = None
        self._f32_cache = {}
        self._ws = None
        self._group_ws = None
        self._sib_out = None
        return super()._apply(fn, *args, **kwargs)

    def packed(self, kinds):
        # the tensor's identity and version too: a buffer replaced by
        # assignment can reuse a freed block's address
        key = (id(self.codes), self.codes.data_ptr(), self.codes._version, self.codes.device, tuple(kinds))
        if self._packed is None or self._packed_key != key:
            if self.codes.is_cuda and torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "QuantizedLinear: the first forward after the module is built, moved, cast or loaded packs "
                    "the codes and reads the scale on the host, which HIP graph capture does not allow: run one "
                    "forward outside capture first")
            self._packed = PackedCodes(self.codes, self.out_features, self.in_features, kinds)
            self._packed_key = key
            self._scale_f = float(self.scale.item())
        return self._packed

    def _fp32(self, name):
        """Buffer ``name`` as float32 for the kernels.  After ``.half()`` or
        ``.to(torch.bfloat16)`` su / sv / bias keep the module's dtype, as in the
        reference, whose forward promotes them to fp32 at use
        (quipsharp/checkpoint.py:141-146); the fp32 copy is made once per buffer
        version.  Under HIP graph capture a missing copy is made uncached: made
        there, it would live in the graph's pool and only be written on replay,
        so an eager call before the first replay would read unwritten memory."""
        t = getattr(self, name)
        if t is None or t.dtype == torch.float32:
            return t
        cache = self.__dict__.setdefault("_f32_cache", {})
        key = (id(t), t.data_ptr(), t._version, t.dtype)
        hit = cache.get(name)
        if hit is None or hit[0] != key:
            if t.is_cuda and torch.cuda.is_current_stream_capturing():
                return t.float().contiguous()
            hit = (key, t.float().contiguous())
            cache[name] = hit
        return hit[1]

    def signs(self, x: Tensor = None):
        """(su, sv) for a forward of x: packed sign bits (a 32nd of the fp32
        bytes, read by every work-group of the transforms) where the library
        takes them (quantize.sign_bits_ok; without x: both sizes on the chunk
        scheme), else the fp32 vectors.  Packed once per sign buffer, outside
        graph capture."""
        from .quantize import sign_bits_ok
        su, sv = self._fp32("su"), self._fp32("sv")
        m, n = self.out_features, self.in_features
        ok = sign_bits_ok(x, m, n) if x is not None else all(d % 256 == 0 and d <= 12288 for d in (m, n))
        if not ok:
            return su, sv
        key = (id(self.su), self.su.data_ptr(), self.su._version, id(self.sv), self.sv.data_ptr(), self.sv._version)
        if getattr(self, "_bits_key", None) != key:
            if torch.cuda.is_current_stream_capturing():
                return su, sv
            from .quantize import pack_signs
            self._bits = (pack_signs(su), pack_signs(sv))
            self._bits_key = key
        return self._bits

    def forward(self, x: Tensor) -> Tensor:
        """quipsharp/checkpoint.py:141-146: y = transform_output(x2 @ W_hat^T) + bias
        in fp32, returned in x.dtype."""
        kinds, s0, s1 = _forward_params(self.codebook, self.num_stages)
        packed = self.packed(kinds)
        if self.transform_kind == "rfft":
            phases = RFFTPhases(phase_u=self.phase_u, phase_v=self.phase_v)
            y = phases.transform_output(decode_matvec(phases.transform_input(x.float()), packed, s0, s1,
                                                      self._scale_f, out_dtype=torch.float32))
            if self.bias is not None:
                y = y + self.bias
            return y.to(x.dtype)
        sib = getattr(self, "_siblings", None)
        if sib is not None and not x.requires_grad and not x.is_inference():
            # linked linears that read the same x: under HIP graph capture the
            # first member called computes the whole group in one grouped
            # forward and leaves each sibling its output, handed out only for
            # this very tensor at this version (an in-place change or another
            # tensor recomputes).  Eager calls stay one per linear: there the
            # host's per-call work, not the GPU, sets the pace, and the grouped
            # call's extra host work made a 7B step 5 % slower, while in a
            # captured step grouping saves 39 %.
            hit = self._sib_out
            self._sib_out = None
            if hit is not None and hit[0]() is x and hit[1] == x._version:
                return hit[2]
            if torch.cuda.is_current_stream_capturing() and groupable(x, sib):
                outs = _grouped(x, sib)
                ref = weakref.ref(x)
                for lin, y in zip(sib, outs):
                    if lin is not self:
                        lin._sib_out = (ref, x._version, y)
                return outs[sib.index(self)]
        return self._forward_one(x)

    def _forward_one(self, x: Tensor) -> Tensor:
        """This linear alone (RHT / Kronecker transforms)."""
        kinds, s0, s1 = _forward_params(self.codebook, self.num_stages)
        packed = self.packed(kinds)
        ws = self._workspace(x, packed)
        su, sv = self.signs(x)
        return forward_packed(x, packed, su, sv, s0, s1, self._scale_f, bias=self._fp32("bias"),
                              out_dtype=x.dtype, workspace=ws)

    def _workspace(self, x, packed):
        from . import _lib
        rows = x.numel() // x.shape[-1] if x.dim() else 1
        need = _lib.lib().qs_linear_workspace_bytes(self.out_features, self.in_features, max(rows, 1), packed.layout)
        if self._ws is None or self._ws.numel() < need or self._ws.device != x.device:
            self._ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=x.device)
        return self._ws


def groupable(x: Tensor, linears) -> bool:
    """True when the library's grouped forward covers these linears for x (rht
    / krht transforms, n a multiple of 256 with n / p >= 256, tiled code
    layout, the same number of stages)."""
    from . import _lib
    from .hadamard import kron_factor
    n = x.shape[-1] if x.dim() else 0
    rows = x.numel() // n if n else 0
    fn = kron_factor(n) if n else None
    if not (1 <= len(linears) <= _lib.QS_MAX_GROUP and rows >= 1 and n % 256 == 0
            and fn is not None and n // fn[0] >= 256):
        return False
    if not all(isinstance(l, QuantizedLinear) and l.transform_kind in ("rht", "krht") and l.in_features == n
               and l.num_stages == linears[0].num_stages for l in linears):
        return False
    for l in linears:
        kinds, _, _ = _forward_params(l.codebook, l.num_stages)
        if l.packed(kinds).layout != _lib.QS_LAYOUT_TILED:
            return False
    return True


def link_sibling_linears(model: nn.Module) -> int:
    """Links the QuantizedLinear modules of each decoder layer that read the
    same input (q/k/v, gate/up: architectures.get_linear_groups), so that
    calling them one by one, as a transformers model does, runs one grouped
    forward per group while a HIP graph is being captured: the first member
    called computes every member's output and the others return theirs (for
    the same input tensor, unchanged).  Outputs are bit-identical to unlinked
    calls.  Returns the number of groups linked.  No counterpart in the
    reference (one linear per call there)."""
    from .architectures import get_decoder_layers, get_linear_groups
    count = 0
    for i, layer in enumerate(get_decoder_layers(model)):
        for group in get_linear_groups(layer, i):
            mods = [m for _, m in group if isinstance(m, QuantizedLinear)]
            if len(mods) == len(group) and len(mods) > 1:
                for m in mods:
                    m._siblings = mods
                    m._sib_out = None
                count += 1
    return count


def grouped_forward(x: Tensor, linears):
    """Outputs of several QuantizedLinear modules that read the same x, as one
    grouped call when the library's grouped forward covers them (rht / krht
    transforms, n a multiple of 256; qs_linear_forward_group: one launch at
    1-2 rows, one launch per stage for the group beyond up to n = 12288, one
    forward per linear above) and one call each otherwise.  Each output equals ``lin(x)``.  No counterpart in the
    reference, which calls the linears one by one; meant for callers that own
    several linears of one input (q/k/v, gate/up)."""
    if not groupable(x, linears):
        return [l._forward_one(x) if isinstance(l, QuantizedLinear) and l.transform_kind != "rfft" else l(x)
                for l in linears]
    return _grouped(x, linears)


def run_preop(x: Tensor, pre: dict) -> Tensor:
    """The rows a pre-operation makes of bf16 x, on their own launch
    (qs_dec_rmsnorm: RMSNorm(x + delta), with x + delta written to h_out)."""
    from . import _lib
    L = _lib.lib()
    n = x.shape[-1]
    rows = x.numel() // n
    xs = x.reshape(rows, n).contiguous()
    out = torch.empty_like(xs)
    stream = _lib.stream_of(xs)
    if pre["kind"] == "rmsnorm":
        delta, h_out = pre.get("delta"), pre.get("h_out")
        d = delta.reshape(rows, n).contiguous() if delta is not None else None
        if d is not None and h_out is None:
            h_out = torch.empty_like(xs)
        o = h_out.reshape(rows, n) if h_out is not None else None
        if o is not None and (not o.is_contiguous() or o.data_ptr() != h_out.data_ptr()):
            raise ValueError("h_out must be contiguous rows")
        _lib.check(L.qs_dec_rmsnorm(_lib.ptr(xs), _lib.ptr(d), _lib.ptr(o), _lib.ptr(pre["weight"]), _lib.ptr(out),
                                    rows, n, n, float(pre.get("eps", 1e-6)), stream))
        if d is None and o is not None:
            o.copy_(xs)  # h' = x: what the pre-operation in the launch writes
    else:
        raise ValueError(f"unknown pre-operation {pre['kind']!r}")
    return out.reshape(x.shape)


def grouped_forward_pre(x: Tensor, linears, pre: dict):
    """``grouped_forward`` on the rows a pre-operation makes of bf16 x
    (``quantize.forward_packed_group``'s ``pre``: RMSNorm with the residual
    add), inside the group's launches where ``quantize.pre_ok`` accepts it
    except at two rows (at one row every work-group of the one-launch kernel
    redoes the norm, which measured faster than the norm's own launch, and
    slower at two; at 3-16 rows the input-transform launch does it once per
    row and linear), otherwise the norm on its own launch first
    (``run_preop``); the outputs are the same either way.  No counterpart in
    the reference, whose decoder runs the norm as a framework kernel before
    each QuantizedLinear.forward."""
    from .quantize import pre_ok
    n = x.shape[-1]
    if x.numel() != 2 * n and groupable(x, linears) and pre_ok(x, n, pre):
        return _grouped(x, linears, pre=pre)
    return grouped_forward(run_preop(x, pre), linears)


def _grouped(x: Tensor, linears, pre: dict = None):
    """The grouped forward proper, for linears that groupable() accepts."""
    from . import _lib
    from .quantize import forward_packed_group
    n = x.shape[-1]
    rows = x.numel() // n
    jobs = []
    signs = [l.signs(x) for l in linears]
    if not all(su.dtype == torch.int32 for su, _ in signs):
        # one sign format per launch: packed bits only when every member has them
        # (a member whose out_features is off the chunk scheme, or whose bits are
        # stale under capture, has fp32 signs)
        signs = [(l._fp32("su"), l._fp32("sv")) for l in linears]
    for l, (su, sv) in zip(linears, signs):
        kinds, s0, s1 = _forward_params(l.codebook, l.num_stages)
        jobs.append((l.packed(kinds), su, sv, s0, s1, l._scale_f, l._fp32("bias")))
    lead = linears[0]
    ms = (ctypes.c_int64 * len(linears))(*[l.out_features for l in linears])
    need = _lib.lib().qs_linear_group_workspace_bytes(n, rows, len(linears), ms)
    ws = getattr(lead, "_group_ws", None)
    if ws is None or ws.numel() < need or ws.device != x.device:
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=x.device)  # zeroed once, reused
        lead._group_ws = ws
    return forward_packed_group(x, jobs, out_dtype=x.dtype, workspace=ws, pre=pre)


def replace_with_quantized_linear_(parent: nn.Module, attr: str, layer: QuantizedLayer, codebook,
                                   bias: Tensor = None) -> QuantizedLinear:
    """quipsharp/checkpoint.py:149-156."""
    qlin = QuantizedLinear.from_quantized_layer(layer, bias=bias)
    qlin.codebook = codebook
    setattr(parent, attr, qlin)
    return qlin


STATE_NAME = "quantized_state.pt"
MANIFEST_NAME = "quip_config.json"


def save_quantized_checkpoint(model: nn.Module, model_id: str, save_path, bits: str, block_size: int, seed: int,
                              quantized_modules: list, tokenizer=None) -> None:
    """quipsharp/checkpoint.py:159-186: the model's state dict (QuantizedLinear
    buffers in the reference's names and dtypes) plus a JSON manifest listing
    every replaced module as {"name", "in_features", "out_features",
    "transform_kind", "has_bias"}."""
    save_path = Path(save_path)
    save_path.mkdir(parents=True, exist_ok=True)
    state = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    torch.save(state, save_path / STATE_NAME)
    manifest = {"model_id": model_id, "bits": bits, "block_size": block_size, "seed": seed,
                "quantized_modules": quantized_modules}
    (save_path / MANIFEST_NAME).write_text(json.dumps(manifest, indent=2))
    if tokenizer is not None:
        tokenizer.save_pretrained(save_path)


def is_quantized_checkpoint(path) -> bool:
    """quipsharp/checkpoint.py:189-190."""
    return (Path(path) / MANIFEST_NAME).exists()


def build_meta_model(model_id, save_path=None) -> nn.Module:
    """The causal-LM architecture for ``model_id`` with its parameters on the
    meta device, in the config's dtype (bf16 if it names none), as
    quipsharp/lazy_weights.py:149-179 builds it: ``get_text_config()`` unwraps multimodal wrappers.  The config
    comes from ``model_id`` when it is a local directory, else from
    ``save_path`` when the checkpoint directory holds a config.json (a copy
    saved beside the checkpoint, for machines without hub access), else from
    the hub / local cache by id."""
    from transformers import AutoConfig, AutoModelForCausalLM
    if Path(str(model_id)).is_dir():
        src = str(model_id)
    elif save_path is not None and (Path(save_path) / "config.json").exists():
        src = str(save_path)
    else:
        src = model_id
    full_config = AutoConfig.from_pretrained(src)
    text_config = full_config.get_text_config()
    dtype = getattr(full_config, "dtype", None) or getattr(full_config, "torch_dtype", None) or torch.bfloat16
    # parameters on the meta device, buffers real (non-persistent ones such as
    # rotary frequencies are not in the saved state), as the reference's
    # accelerate.init_empty_weights() does
    from accelerate import init_empty_weights
    with init_empty_weights():
        model = AutoModelForCausalLM.from_config(text_config, dtype=dtype)
    return model


def install_quantized_placeholders(model: nn.Module, manifest: dict) -> None:
    """Swaps an empty QuantizedLinear of the recorded shape, transform, stage
    count and bias into ``model`` at every module the manifest lists
    (quipsharp/checkpoint.py:216-223), ready for ``load_state_dict``."""
    stages = num_rvq_stages(manifest["bits"])
    for info in manifest["quantized_modules"]:
        parent_name, _, attr = info["name"].rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        qlin = QuantizedLinear(info["in_features"], info["out_features"], manifest["block_size"],
                               info["transform_kind"], num_stages=stages, has_bias=info.get("has_bias", False))
        setattr(parent, attr, qlin)


def checkpoint_placement(total_bytes, device="cuda", gpu_devices=None, gpu_budget_bytes=None,
                         cpu_budget_bytes=0):
    """The device a checkpoint of ``total_bytes`` loads onto, and a warning
    (or None).  The reference (quipsharp/checkpoint.py:228-263) puts
    everything on ``gpu_devices[0]`` (else ``device``) when it fits
    ``gpu_budget_bytes``, and otherwise bin-packs the decoder layers over
    ``gpu_devices``, then the CPU when ``cpu_budget_bytes`` is nonzero, the
    last device taking what is left.  Here the forward runs on one GPU and has
    no CPU path: with one GPU listed the whole model goes on it (with no CPU
    budget that is where the reference's packing ends as well; with one, the
    layers it would have put on the CPU stay on the GPU, and the warning says
    so); with several GPUs listed and a checkpoint above the budget,
    NotImplementedError names the two ways out (one device, or a larger
    budget: an MI355X holds 288 GB)."""
    if gpu_devices is None or gpu_budget_bytes is None or total_bytes <= gpu_budget_bytes:
        return (gpu_devices[0] if gpu_devices else device), None
    gpus = list(gpu_devices)
    if len(gpus) == 1:
        where = (" (the reference would put the layers past the budget on the CPU; the forward here runs on the "
                 "GPU only)") if cpu_budget_bytes else ""
        return gpus[0], (f"the checkpoint holds {total_bytes} bytes, more than gpu_budget_bytes={gpu_budget_bytes}: "
                         f"all of it goes on {gpus[0]}{where}")
    raise NotImplementedError(
        f"the checkpoint holds {total_bytes} bytes, more than gpu_budget_bytes={gpu_budget_bytes}, and "
        f"{len(gpus)} devices are listed: spreading layers over several devices (accelerate.dispatch_model in the "
        "reference) is not implemented; pass one device in gpu_devices, or a gpu_budget_bytes of at least the "
        "checkpoint's size")


def load_quantized_checkpoint(save_path, device="cuda", gpu_devices=None, gpu_budget_bytes=None,
                              cpu_budget_bytes=0, model: nn.Module = None) -> nn.Module:
    """quipsharp/checkpoint.py:193-275, same call (quipsharp/model_loading.py:57
    passes ``device``, ``gpu_devices``, ``gpu_budget_bytes``,
    ``cpu_budget_bytes``): the architecture skeleton is built on the meta
    device from the manifest's model id (``build_meta_model``; or pass
    ``model``, a skeleton built by the caller), every manifest entry becomes an
    empty QuantizedLinear of the recorded shape and transform, the saved state
    dict is loaded with ``assign=True`` through ``torch.load(weights_only=True)``
    (tensors only, nothing executed from the file), the model moves to
    ``gpu_devices[0]`` (or ``device``) and each QuantizedLinear gets the
    codebook rebuilt from the manifest's bits and seed.  Placement for a
    checkpoint larger than ``gpu_budget_bytes``: see ``checkpoint_placement``."""
    save_path = Path(save_path)
    manifest = json.loads((save_path / MANIFEST_NAME).read_text())
    state = torch.load(save_path / STATE_NAME, map_location="cpu", weights_only=True)
    total_bytes = sum(t.numel() * t.element_size() for t in state.values())
    device, note = checkpoint_placement(total_bytes, device, gpu_devices, gpu_budget_bytes, cpu_budget_bytes)
    if note:
        warnings.warn(note, stacklevel=2)
    if model is None:
        model = build_meta_model(manifest["model_id"], save_path)
    install_quantized_placeholders(model, manifest)
    model.load_state_dict(state, strict=True, assign=True)
    model.to(device)
    codebook, _ = build_codebook(manifest["bits"], device, manifest["seed"])
    for info in manifest["quantized_modules"]:
        model.get_submodule(info["name"]).codebook = codebook
    model.eval()
    try:
        link_sibling_linears(model)  # q/k/v and gate/up called one by one run grouped
    except (AttributeError, NotImplementedError, ValueError):
        pass  # an architecture without the standard decoder layout: linears stay independent
    return model
