"""The drop-in surface without a GPU: the reference's import root
(``quipsharp``) resolves to this library's modules, and a checkpoint written
by the reference's own save path (tests/golden/ref_ckpt, made by
tests/golden/make_golden.py from quipsharp/checkpoint.py:149-186) loads into
the architecture skeleton with every key matched."""
import json
import os

import pytest
import torch

from conftest import GOLDEN

CKPT = os.path.join(GOLDEN, "ref_ckpt")


def test_quipsharp_import_root_aliases_the_library():
    import quipsharp
    import quipsharp_amd
    from quipsharp.checkpoint import (QuantizedLinear, build_codebook, is_quantized_checkpoint,  # noqa: F401
                                      load_quantized_checkpoint, replace_with_quantized_linear_,
                                      save_quantized_checkpoint)
    from quipsharp.model_loading import load_eval_model, resolve_cpu_budget_bytes, resolve_gpu_budget_bytes  # noqa
    from quipsharp.quantize import dequantize_linear, linear_forward, quantize_linear  # noqa: F401
    from quipsharp.codebooks.e8p import E8PCodebook  # noqa: F401
    import importlib
    for name in ("hadamard", "incoherence", "rfft", "rvq", "ldlq", "quantize", "checkpoint", "model_loading"):
        assert getattr(quipsharp, name) is importlib.import_module("quipsharp_amd." + name)
        assert importlib.import_module("quipsharp." + name) is importlib.import_module("quipsharp_amd." + name)
    assert quipsharp.checkpoint is quipsharp_amd.checkpoint
    assert resolve_gpu_budget_bytes("2") == 2 * 1024 ** 3 and resolve_cpu_budget_bytes("0.5") == 512 * 1024 ** 2


def test_reference_checkpoint_keys_match():
    """Every tensor of the reference-written state dict lands in a buffer of
    the same name, shape and dtype (load_state_dict strict, on the meta
    skeleton built from the manifest's model id / the saved config)."""
    from quipsharp_amd.checkpoint import (MANIFEST_NAME, STATE_NAME, QuantizedLinear, build_meta_model,
                                          install_quantized_placeholders, is_quantized_checkpoint)
    assert is_quantized_checkpoint(CKPT)
    manifest = json.loads(open(os.path.join(CKPT, MANIFEST_NAME)).read())
    state = torch.load(os.path.join(CKPT, STATE_NAME), map_location="cpu", weights_only=True)
    model = build_meta_model(manifest["model_id"], CKPT)
    install_quantized_placeholders(model, manifest)
    want = {k: (tuple(v.shape), v.dtype) for k, v in model.state_dict().items()}
    got = {k: (tuple(v.shape), v.dtype) for k, v in state.items()}
    assert want == got
    model.load_state_dict(state, strict=True, assign=True)
    kinds = {m["name"]: m["transform_kind"] for m in manifest["quantized_modules"]}
    assert set(kinds.values()) == {"rht", "rfft"}
    for name, kind in kinds.items():
        mod = model.get_submodule(name)
        assert isinstance(mod, QuantizedLinear) and mod.transform_kind == kind
        assert mod.codes.dtype == torch.int16 and mod.codes.device.type == "cpu"


def test_multi_device_split_refused():
    """A checkpoint above gpu_budget_bytes with several GPUs listed (the
    reference spreads it over them with accelerate) is refused before anything
    is placed; with one GPU listed it would go there whole (a warning)."""
    from quipsharp_amd.checkpoint import load_quantized_checkpoint
    with pytest.raises(NotImplementedError, match="pass one device"):
        load_quantized_checkpoint(CKPT, device="cuda:0", gpu_devices=["cuda:0", "cuda:1"], gpu_budget_bytes=1)
