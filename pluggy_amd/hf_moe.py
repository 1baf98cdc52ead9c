"""Hugging Face checkpoint import and export of Qwen3-MoE expert weights.

The reference's importer (pluggy/models/hf_import.py:72-99) maps dense Qwen3
keys only: a hub Qwen3-MoE checkpoint stores every expert as separate tensors,

    model.layers.{l}.mlp.gate.weight                      (E, H)  router
    model.layers.{l}.mlp.experts.{e}.gate_proj.weight     (I, H)
    model.layers.{l}.mlp.experts.{e}.up_proj.weight       (I, H)
    model.layers.{l}.mlp.experts.{e}.down_proj.weight     (H, I)

while ``Qwen3MoeSparseMLP`` packs them per layer (qwen3_moe.py:181-231):

    blocks.{l}.ffn.router.weight                          (E, H)
    blocks.{l}.ffn.experts.gate_up_proj                   (E, 2I, H)  rows [0, I) gate, [I, 2I) up
    blocks.{l}.ffn.experts.down_proj                      (E, H, I)

(the gate-first packing is the ``chunk(2)`` order of pluggy/kernels/moe.py:117).
``pack_moe_state`` turns the former into the latter and hands back every
non-MoE key untouched, for the reference's dense mapping (``hf_to_local``);
``unpack_moe_state`` is its inverse. Files are read with the ``safetensors``
package (no code in the file is executed). Like the reference importer, every
mismatch is loud: a missing expert or projection, an expert id past E, an
unknown MoE key or a shape disagreement raises.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

import torch

_EXPERT = re.compile(r"model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\.weight")
_ROUTER = re.compile(r"model\.layers\.(\d+)\.mlp\.gate\.weight")
_MOE_ANY = re.compile(r"model\.layers\.(\d+)\.mlp\.(gate\.|experts\.|shared_expert)")


def weight_files(directory: str | Path) -> list[Path]:
    """safetensors files of a local checkpoint directory (single file or index-sharded).

    Same resolution as pluggy/models/hf_import.py:102-132 for a local directory;
    hub ids are not fetched (no network here).
    """
    d = Path(directory)
    index = d / "model.safetensors.index.json"
    if index.exists():
        with open(index) as f:
            shards = sorted(set(json.load(f)["weight_map"].values()))
        return [d / s for s in shards]
    single = d / "model.safetensors"
    assert single.exists(), f"{d} has neither model.safetensors nor model.safetensors.index.json"
    return [single]


def read_state(directory: str | Path) -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    state: dict[str, torch.Tensor] = {}
    for path in weight_files(directory):
        state.update(load_file(str(path)))
    return state


def pack_moe_state(state: dict[str, torch.Tensor], prefix: str = "blocks.{layer}.ffn.") -> tuple[
        dict[str, torch.Tensor], dict[str, torch.Tensor]]:
    """HF per-expert tensors -> packed ``Qwen3MoeSparseMLP`` tensors.

    Returns ``(packed, rest)``: ``packed`` maps ``prefix``-formatted names to the
    router weight and the packed expert tensors of every MoE layer found;
    ``rest`` holds every key that is not part of an MoE layer.
    """
    experts: dict[int, dict[int, dict[str, torch.Tensor]]] = {}
    routers: dict[int, torch.Tensor] = {}
    rest: dict[str, torch.Tensor] = {}
    for name, t in state.items():
        m = _EXPERT.fullmatch(name)
        if m:
            layer, e, proj = int(m.group(1)), int(m.group(2)), m.group(3)
            experts.setdefault(layer, {}).setdefault(e, {})[proj] = t
            continue
        m = _ROUTER.fullmatch(name)
        if m:
            routers[int(m.group(1))] = t
            continue
        assert not _MOE_ANY.match(name), f"unsupported MoE key {name} (shared experts are not part of Qwen3-MoE)"
        rest[name] = t

    packed: dict[str, torch.Tensor] = {}
    layers = sorted(set(experts) | set(routers))
    for layer in layers:
        assert layer in routers, f"layer {layer}: experts without a router (mlp.gate.weight)"
        assert layer in experts, f"layer {layer}: a router without experts"
        router = routers[layer]
        E, H = router.shape
        ex = experts[layer]
        assert sorted(ex) == list(range(E)), (
            f"layer {layer}: router has {E} experts but the checkpoint holds expert ids "
            f"{sorted(ex)[:8]}{'...' if len(ex) > 8 else ''}")
        gate_up, down = [], []
        for e in range(E):
            proj = ex[e]
            missing = {"gate_proj", "up_proj", "down_proj"} - set(proj)
            assert not missing, f"layer {layer} expert {e}: missing {sorted(missing)}"
            g, u, d = proj["gate_proj"], proj["up_proj"], proj["down_proj"]
            I = g.shape[0]
            assert g.shape == (I, H) and u.shape == (I, H), (
                f"layer {layer} expert {e}: gate {tuple(g.shape)} / up {tuple(u.shape)}, expected ({I}, {H})")
            assert d.shape == (H, I), f"layer {layer} expert {e}: down {tuple(d.shape)}, expected ({H}, {I})"
            if e:
                assert I == gate_up[0].shape[0] // 2, f"layer {layer} expert {e}: intermediate size {I} differs"
            gate_up.append(torch.cat([g, u], dim=0))
            down.append(d)
        p = prefix.format(layer=layer)
        packed[p + "router.weight"] = router
        packed[p + "experts.gate_up_proj"] = torch.stack(gate_up)
        packed[p + "experts.down_proj"] = torch.stack(down)
    return packed, rest


def unpack_moe_state(packed: dict[str, torch.Tensor], prefix: str = "blocks.{layer}.ffn.") -> dict[str, torch.Tensor]:
    """Inverse of ``pack_moe_state``: packed module tensors -> HF per-expert names."""
    pat = re.compile(re.escape(prefix).replace(r"\{layer\}", r"(\d+)") + r"(router\.weight|experts\.gate_up_proj|"
                     r"experts\.down_proj)")
    out: dict[str, torch.Tensor] = {}
    for name, t in packed.items():
        m = pat.fullmatch(name)
        assert m, f"not a packed MoE tensor name: {name}"
        layer, what = int(m.group(1)), m.group(2)
        base = f"model.layers.{layer}.mlp."
        if what == "router.weight":
            out[base + "gate.weight"] = t
        elif what == "experts.gate_up_proj":
            I = t.shape[1] // 2
            for e in range(t.shape[0]):
                out[base + f"experts.{e}.gate_proj.weight"] = t[e, :I].contiguous()
                out[base + f"experts.{e}.up_proj.weight"] = t[e, I:].contiguous()
        else:
            for e in range(t.shape[0]):
                out[base + f"experts.{e}.down_proj.weight"] = t[e].contiguous()
    return out


def load_hf_moe_weights(model: torch.nn.Module, directory: str | Path,
                        prefix: str = "blocks.{layer}.ffn.") -> tuple[int, dict[str, torch.Tensor]]:
    """Copy the MoE layers of a local HF Qwen3-MoE checkpoint into ``model`` in place.

    Parameters keep their device and dtype (bf16 hub weights land in fp32
    masters, as pluggy/models/hf_import.py:135-171). Returns ``(number of packed
    tensors loaded, the remaining non-MoE tensors)`` — the latter go through the
    reference's dense mapping.
    """
    packed, rest = pack_moe_state(read_state(directory), prefix)
    model_sd = model.state_dict()
    for name, t in packed.items():
        assert name in model_sd, f"packed key {name} not in the model"
        assert model_sd[name].shape == t.shape, (
            f"{name}: checkpoint {tuple(t.shape)} vs model {tuple(model_sd[name].shape)} -- the model's "
            f"emb_dim / moe_ffn_dim / num_experts must match the hub config")
    with torch.no_grad():
        for name, t in packed.items():
            model_sd[name].copy_(t.to(model_sd[name].dtype))
    return len(packed), rest
