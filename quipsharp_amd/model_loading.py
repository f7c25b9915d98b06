"""The loading entry point the reference's evaluation scripts call
(quipsharp/model_loading.py; scripts/eval_ppl.py:18, eval_zeroshot.py),
for this library's compact quantized checkpoints on one GPU.

``load_eval_model`` returns ``(model, main_device)`` like the reference.  A
directory holding a quantized checkpoint loads through
``checkpoint.load_quantized_checkpoint``; any other model (a dense baseline)
loads with ``transformers``' ``from_pretrained`` onto the first device.
Spreading a model over several devices or offloading to the CPU (the
reference's accelerate paths) is not implemented: this library runs on one
GPU."""
from pathlib import Path

from .checkpoint import is_quantized_checkpoint, load_quantized_checkpoint


_GIB = 1 << 30


def _gib(arg) -> int:
    return int(float(arg) * _GIB)


def resolve_gpu_budget_bytes(arg, headroom_frac: float = 0.15) -> int:
    """quipsharp/model_loading.py:12-22 (same meaning): a number is a size in
    GiB; "auto" is what the tightest visible GPU can still take -- its free
    bytes less ``headroom_frac`` of its capacity (0 with no GPU)."""
    if arg != "auto":
        return _gib(arg)
    import torch
    best = None
    for dev in range(torch.cuda.device_count()):
        free, capacity = torch.cuda.mem_get_info(dev)
        room = free - int(capacity * headroom_frac)
        best = room if best is None else min(best, room)
    return best or 0


def _host_available_bytes() -> int:
    """MemAvailable of /proc/meminfo, in bytes."""
    for line in Path("/proc/meminfo").read_text().splitlines():
        key, _, rest = line.partition(":")
        if key == "MemAvailable":
            return int(rest.split()[0]) * 1024
    raise RuntimeError("/proc/meminfo has no MemAvailable line")


def resolve_cpu_budget_bytes(arg, use_frac: float = 0.8) -> int:
    """quipsharp/model_loading.py:25-33 (same meaning): a number is a size in
    GiB; "auto" is ``use_frac`` of the host memory available now."""
    if arg != "auto":
        return _gib(arg)
    return int(_host_available_bytes() * use_frac)


def load_eval_model(model_id_or_path: str, gpu_devices=("cuda:0",), gpu_budget_bytes: int = 20 * 1024 ** 3,
                    cpu_budget_bytes: int = 60 * 1024 ** 3, offload_folder: str = None):
    """quipsharp/model_loading.py:36-96 for one device: (model, main_device)."""
    main_device = gpu_devices[0] if gpu_devices else "cpu"
    if Path(model_id_or_path).is_dir() and is_quantized_checkpoint(model_id_or_path):
        model = load_quantized_checkpoint(model_id_or_path, device=main_device, gpu_devices=list(gpu_devices),
                                          gpu_budget_bytes=gpu_budget_bytes, cpu_budget_bytes=cpu_budget_bytes)
        return model, main_device
    from transformers import AutoModelForCausalLM
    model = AutoModelForCausalLM.from_pretrained(model_id_or_path, dtype="auto", low_cpu_mem_usage=True)
    model.to(main_device).eval()
    return model, main_device
