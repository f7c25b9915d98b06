"""GPU: a checkpoint written by the reference's own save path
(tests/golden/ref_ckpt: quipsharp/checkpoint.py:149-186 on a one-layer
Llama-shaped model with "rht" layers at 256 and "rfft" layers at 384) loads
through load_quantized_checkpoint with the reference's call
(quipsharp/model_loading.py:57) and through the reference's entry point
load_eval_model (scripts/eval_ppl.py:18), and reproduces the reference's CPU
forward: each quantized module within 1e-3 (relative, norm-wise; fp32
accumulation), the model's logits within 5e-3."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, golden

pytestmark = pytest.mark.gpu

CKPT = os.path.join(GOLDEN, "ref_ckpt")


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def loaded(dev):
    from quipsharp_amd.checkpoint import load_quantized_checkpoint
    return load_quantized_checkpoint(CKPT, device=str(dev), gpu_devices=None, gpu_budget_bytes=None,
                                     cpu_budget_bytes=0)


def test_modules_match_reference_forward(dev, loaded):
    import json
    from quipsharp_amd.checkpoint import QuantizedLinear
    ref = golden("ref_ckpt_outputs.npz")
    manifest = json.loads(open(os.path.join(CKPT, "quip_config.json")).read())
    for info in manifest["quantized_modules"]:
        mod = loaded.get_submodule(info["name"])
        assert isinstance(mod, QuantizedLinear) and mod.transform_kind == info["transform_kind"]
        key = info["name"].replace(".", "_")
        x = torch.from_numpy(ref[key + "_x"]).to(dev)
        with torch.no_grad():
            y = mod(x).cpu().numpy()
        err = rel(y, ref[key + "_y"])
        print(f"{info['name']} ({info['transform_kind']}): relative difference {err:.2e}", flush=True)
        assert err < 1e-3, (info["name"], err)


def test_logits_match_reference(dev, loaded):
    ref = golden("ref_ckpt_outputs.npz")
    with torch.no_grad():
        logits = loaded(torch.from_numpy(ref["ids"]).to(dev)).logits.float().cpu().numpy()
    err = rel(logits, ref["logits"])
    print(f"logits relative difference {err:.2e}", flush=True)
    assert err < 5e-3


def test_eval_entry_point_loads_the_same_model(dev, loaded):
    """scripts/eval_ppl.py's import, unchanged: quipsharp.model_loading."""
    from quipsharp.model_loading import load_eval_model
    model, main_device = load_eval_model(CKPT, gpu_devices=(str(dev),), gpu_budget_bytes=1 << 34)
    assert main_device == str(dev)
    ids = torch.from_numpy(golden("ref_ckpt_outputs.npz")["ids"]).to(dev)
    with torch.no_grad():
        a = model(ids).logits
        b = loaded(ids).logits
    assert torch.allclose(a, b, rtol=1e-5, atol=1e-5)
