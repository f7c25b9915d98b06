"""The decode harness on a tiny Qwen3-shaped model: linear discovery, random
quantized layers, logits against the same model with dense reconstructed
weights, and a few greedy KV-cache steps."""
import copy

import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu


def _tiny_config():
    from transformers import Qwen3Config
    return Qwen3Config(hidden_size=512, intermediate_size=1536, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=2, head_dim=128, vocab_size=1000, tie_word_embeddings=False,
                       max_position_embeddings=512)


def test_linear_groups_of_qwen3():
    from transformers import Qwen3ForCausalLM
    from quipsharp_amd.architectures import get_decoder_layers, get_linear_groups
    with torch.device("meta"):
        model = Qwen3ForCausalLM(_tiny_config())
    groups = get_linear_groups(get_decoder_layers(model)[0], 0)
    assert [[n for n, _ in g] for g in groups] == [
        ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"], ["self_attn.o_proj"],
        ["mlp.gate_proj", "mlp.up_proj"], ["mlp.down_proj"]]


def test_quantized_model_matches_dense_reconstruction(dev):
    from quipsharp_amd.checkpoint import QuantizedLinear
    from quipsharp_amd.decode import greedy_decode, random_quantized_model
    from quipsharp_amd.quantize import dequantize_linear
    cfg = _tiny_config()
    model = random_quantized_model(cfg, dev, seed=0)
    kinds = {type(m).__name__ for m in model.modules()}
    assert "QuantizedLinear" in kinds and not any(isinstance(m, nn.Linear) and m.in_features == 512
                                                  for m in model.model.layers.modules())
    dense = copy.deepcopy(model)
    for name, mod in list(dense.named_modules()):
        if isinstance(mod, QuantizedLinear):
            layer = mod._quantized_layer()
            W = layer.signs.reconstruct_weight(dequantize_linear(layer, mod.codebook))
            lin = nn.Linear(mod.in_features, mod.out_features, bias=False, device=dev, dtype=torch.float32)
            lin.weight.data.copy_(W)
            lin.to(torch.bfloat16)
            parent, _, attr = name.rpartition(".")
            setattr(dense.get_submodule(parent), attr, lin)
    ids = torch.randint(0, cfg.vocab_size, (2, 24), generator=torch.Generator().manual_seed(0)).to(dev)
    with torch.no_grad():
        a = model(input_ids=ids).logits.float()
        b = dense(input_ids=ids).logits.float()
    rel = ((a - b).norm() / b.norm()).item()
    assert rel < 3e-2, rel
    toks, pre, dec = greedy_decode(model, ids, 4)
    assert toks.shape == (2, 4) and pre > 0 and dec > 0


def test_static_decoder_matches_transformers(dev):
    """StaticDecoder's logits follow the transformers forward with a dynamic
    cache (prefill and decode steps), and the HIP-graph replay of its decode
    step gives exactly its eager tokens."""
    from transformers import DynamicCache
    from quipsharp_amd.decode import StaticDecoder, greedy_decode_static, random_quantized_model
    cfg = _tiny_config()
    model = random_quantized_model(cfg, dev, seed=1)
    ids = torch.randint(0, cfg.vocab_size, (2, 16), generator=torch.Generator().manual_seed(1)).to(dev)
    dec = StaticDecoder(model, 2, 32)
    cache = DynamicCache()
    with torch.no_grad():
        ref = model(input_ids=ids, past_key_values=cache, use_cache=True).logits[:, -1].float()
        got = dec.step(ids, torch.arange(16, device=dev)).float()
        assert ((got - ref).norm() / ref.norm()).item() < 2e-2
        tok = ref.argmax(-1, keepdim=True)
        for p in range(16, 20):
            ref = model(input_ids=tok, past_key_values=cache, use_cache=True).logits[:, -1].float()
            got = dec.step(tok, torch.full((1,), p, dtype=torch.long, device=dev)).float()
            assert ((got - ref).norm() / ref.norm()).item() < 2e-2, p
            tok = ref.argmax(-1, keepdim=True)
    a, _, _ = greedy_decode_static(model, ids, 8, use_graph=False)
    b, _, _ = greedy_decode_static(model, ids, 8)
    assert torch.equal(a, b)


@pytest.mark.parametrize("rows", [1, 2, 3])
def test_grouped_forward_equals_separate_calls(dev, rows):
    """checkpoint.grouped_forward: one launch for q/k/v (and gate/up) at 1-2
    rows, bit-identical to calling the modules one by one; one call each
    beyond."""
    from quipsharp_amd.architectures import get_decoder_layers
    from quipsharp_amd.checkpoint import grouped_forward
    from quipsharp_amd.decode import random_quantized_model
    model = random_quantized_model(_tiny_config(), dev, seed=3)
    layer = get_decoder_layers(model)[0]
    x = torch.randn(rows, 512, generator=torch.Generator().manual_seed(rows)).to(dev).bfloat16()
    with torch.no_grad():
        for mods in ([layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj],
                     [layer.mlp.gate_proj, layer.mlp.up_proj]):
            got = grouped_forward(x, mods)
            want = [m(x) for m in mods]
            assert len(got) == len(want)
            for g_, w_ in zip(got, want):
                assert g_.dtype == w_.dtype and torch.equal(g_, w_)


@pytest.mark.parametrize("rows", [1, 16])
def test_linked_siblings_called_one_by_one(dev, rows, monkeypatch):
    """link_sibling_linears: q/k/v (and gate/up) called one by one, as a
    transformers model does, run one grouped forward per group; every output
    is bit-identical to the unlinked call, and an input changed in place or a
    different tensor is recomputed, never served from the group's results."""
    from quipsharp_amd import quantize
    from quipsharp_amd.architectures import get_decoder_layers
    from quipsharp_amd.decode import random_quantized_model
    model = random_quantized_model(_tiny_config(), dev, seed=4)
    layer = get_decoder_layers(model)[0]
    mods = [layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj]
    assert all(m._siblings is mods[0]._siblings for m in mods) and len(mods[0]._siblings) == 3
    x = torch.randn(rows, 512, generator=torch.Generator().manual_seed(rows)).to(dev).bfloat16()
    with torch.no_grad():
        want = [m._forward_one(x) for m in mods]
        calls = {"group": 0}
        real = quantize.forward_packed_group

        def counting(*a, **k):
            calls["group"] += 1
            return real(*a, **k)
        monkeypatch.setattr(quantize, "forward_packed_group", counting)
        # eager: one call per linear, no grouping
        got = [m(x) for m in mods]
        assert calls["group"] == 0
        for g_, w_ in zip(got, want):
            assert torch.equal(g_, w_)
        # captured: the first member computes the group, the others take theirs
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            [m(x) for m in mods]
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            got = [m(x) for m in mods]
        assert calls["group"] == 1
        for rep in range(3):
            for g_ in got:
                g_.zero_()
            graph.replay()
            torch.cuda.synchronize()
            for g_, w_ in zip(got, want):
                assert torch.equal(g_, w_), rep
        del graph
        monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)  # group eagerly from here on
        calls["group"] = 0
        got = [m(x) for m in mods]
        assert calls["group"] == 1
        for g_, w_ in zip(got, want):
            assert torch.equal(g_, w_)
        # q again recomputes the group; an in-place change of x before k does too
        mods[0](x)
        x.mul_(2.0)
        k2 = mods[1](x)
        assert torch.equal(k2, mods[1]._forward_one(x))
        # a different tensor with the same values is not served from the group of x
        mods[0](x)
        x2 = x.clone()
        assert torch.equal(mods[2](x2), mods[2]._forward_one(x2))
