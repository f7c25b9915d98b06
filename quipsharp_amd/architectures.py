"""Decoder-layer and linear-group discovery (quipsharp/architectures.py:27-94):
the Llama / Qwen2.5 / Qwen3 / Gemma families all name their linears
self_attn.{q,k,v,o}_proj and mlp.{gate,up,down}_proj, so one
attribute-presence walk covers them; MoE blocks are refused."""
from torch import nn


class MoEUnsupportedError(NotImplementedError):
    """A decoder layer with expert routing (expert weights are not nn.Linear)."""


def get_decoder_layers(model) -> list:
    """quipsharp/architectures.py:27-30."""
    return list(model.model.layers)


def get_model_dims(config) -> tuple:
    """quipsharp/architectures.py:33-37: (layers, hidden, intermediate)."""
    return config.num_hidden_layers, config.hidden_size, config.intermediate_size


def _check_no_moe(layer, layer_index):
    mlp = getattr(layer, "mlp", None)
    if mlp is not None and (hasattr(mlp, "experts") or hasattr(mlp, "router")):
        raise MoEUnsupportedError(f"layer {layer_index}: mlp has experts/router (MoE) -- not supported")
    if hasattr(layer, "router") or hasattr(layer, "experts"):
        raise MoEUnsupportedError(f"layer {layer_index}: has router/experts (MoE) -- not supported")


def get_linear_groups(layer, layer_index: int = -1) -> list:
    """quipsharp/architectures.py:52-94: the layer's linears grouped by shared
    input -- [q,k,v] (those present), [o], [gate,up], [down] -- as
    (relative name, module) pairs.  Accepts nn.Linear and modules that
    already replaced one (anything with in_features / out_features)."""
    _check_no_moe(layer, layer_index)

    def is_linear(mod):
        return isinstance(mod, nn.Linear) or (mod is not None and hasattr(mod, "in_features")
                                              and hasattr(mod, "out_features"))

    groups = []
    attn = getattr(layer, "self_attn", None)
    if attn is not None:
        qkv = [(f"self_attn.{k}", getattr(attn, k)) for k in ("q_proj", "k_proj", "v_proj")
               if is_linear(getattr(attn, k, None))]
        if qkv:
            groups.append(qkv)
        if is_linear(getattr(attn, "o_proj", None)):
            groups.append([("self_attn.o_proj", attn.o_proj)])
    mlp = getattr(layer, "mlp", None)
    if mlp is not None:
        gu = [(f"mlp.{k}", getattr(mlp, k)) for k in ("gate_proj", "up_proj") if is_linear(getattr(mlp, k, None))]
        if gu:
            groups.append(gu)
        if is_linear(getattr(mlp, "down_proj", None)):
            groups.append([("mlp.down_proj", mlp.down_proj)])
    return groups
