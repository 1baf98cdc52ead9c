"""HF Qwen3-MoE checkpoint import/export of the packed expert tensors (CPU).

The checkpoints are written by transformers' own ``save_pretrained`` (hub layout:
one tensor per expert and projection), so the packing is checked against an
implementation independent of ``pluggy_amd.hf_moe``: transformers' in-memory
``experts.gate_up_proj`` / ``down_proj`` must come out bitwise, and transformers'
``Qwen3MoeSparseMoeBlock`` forward must agree with the oracle's block on the
imported weights (this also pins the oracle's router + FFN against that
independent implementation). Error paths mirror the reference importer's loud
failures (tests/hf_import.py in the reference).
"""

from __future__ import annotations

import json
import os

import pytest
import torch
from safetensors.torch import load_file, save_file

from oracle import moe_oracle as om
from pluggy_amd import Qwen3MoeSparseMLP
from pluggy_amd.hf_moe import load_hf_moe_weights, pack_moe_state, read_state, unpack_moe_state, weight_files

H, I, E, K, L = 16, 8, 6, 2, 2


def _hf_model(seed: int = 0):
    os.environ.setdefault("HF_HUB_OFFLINE", "1")
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3MoeConfig(
        vocab_size=32, hidden_size=H, intermediate_size=24, moe_intermediate_size=I, num_hidden_layers=L,
        num_attention_heads=2, num_key_value_heads=1, head_dim=8, num_experts=E, num_experts_per_tok=K,
        norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[], tie_word_embeddings=False)
    torch.manual_seed(seed)
    m = transformers.Qwen3MoeForCausalLM(cfg)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.5)
    return m


class _Blocks(torch.nn.Module):
    """Stand-in for the reference model's ``blocks`` list (qwen3_moe.py:371) holding the drop-in FFNs."""

    class _Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.ffn = Qwen3MoeSparseMLP(H, I, E, K, True)

    def __init__(self, n: int = L):
        super().__init__()
        self.blocks = torch.nn.ModuleList(self._Block() for _ in range(n))


@pytest.fixture(scope="module")
def hub(tmp_path_factory):
    m = _hf_model()
    single = tmp_path_factory.mktemp("single")
    m.save_pretrained(single)
    sharded = tmp_path_factory.mktemp("sharded")
    m.save_pretrained(sharded, max_shard_size="4KB")
    return m, single, sharded


def test_pack_matches_transformers_layout(hub):
    m, single, sharded = hub
    assert len(weight_files(single)) == 1
    assert len(weight_files(sharded)) > 2
    sd = m.state_dict()
    for d in (single, sharded):
        packed, rest = pack_moe_state(read_state(d))
        assert len(packed) == 3 * L
        for layer in range(L):
            hf = f"model.layers.{layer}.mlp."
            p = f"blocks.{layer}.ffn."
            assert torch.equal(packed[p + "router.weight"], sd[hf + "gate.weight"])
            assert torch.equal(packed[p + "experts.gate_up_proj"], sd[hf + "experts.gate_up_proj"])
            assert torch.equal(packed[p + "experts.down_proj"], sd[hf + "experts.down_proj"])
        assert not any(".mlp." in k for k in rest)
        assert "model.embed_tokens.weight" in rest and "model.layers.1.self_attn.q_proj.weight" in rest


def test_unpack_is_inverse_of_pack(hub):
    _, single, _ = hub
    hub_state = load_file(str(single / "model.safetensors"))
    packed, rest = pack_moe_state(hub_state)
    back = unpack_moe_state(packed)
    assert set(back) | set(rest) == set(hub_state)
    for k, t in back.items():
        assert torch.equal(t, hub_state[k]), k


def test_load_into_dropin_and_block_forward(hub):
    m, single, _ = hub
    model = _Blocks()
    n, rest = load_hf_moe_weights(model, single)
    assert n == 3 * L and "lm_head.weight" in rest
    g = torch.Generator().manual_seed(1)
    for layer in range(L):
        ffn = model.blocks[layer].ffn
        hf_block = m.model.layers[layer].mlp
        x = torch.randn(2, 5, H, generator=g)
        with torch.no_grad():
            want = hf_block(x)
            got, logits = om.sparse_mlp_forward(x, ffn.router.weight, ffn.experts.gate_up_proj,
                                                ffn.experts.down_proj, K, True)
        assert om.rel_l2(got, want) < 1e-6
        assert torch.allclose(logits, x.reshape(-1, H) @ hf_block.gate.weight.T, rtol=1e-5, atol=1e-6)


def test_bf16_checkpoint_into_fp32_masters(tmp_path, hub):
    _, single, _ = hub
    state = {k: v.to(torch.bfloat16) for k, v in read_state(single).items()}
    save_file(state, str(tmp_path / "model.safetensors"))
    model = _Blocks()
    load_hf_moe_weights(model, tmp_path)
    p = model.blocks[0].ffn.experts.gate_up_proj
    assert p.dtype == torch.float32
    assert torch.equal(p[3, :I], state["model.layers.0.mlp.experts.3.gate_proj.weight"].float())
    assert torch.equal(p[3, I:], state["model.layers.0.mlp.experts.3.up_proj.weight"].float())


def _state():
    g = torch.Generator().manual_seed(2)
    s = {"model.layers.0.mlp.gate.weight": torch.randn(E, H, generator=g),
         "model.norm.weight": torch.ones(H)}
    for e in range(E):
        b = f"model.layers.0.mlp.experts.{e}."
        s[b + "gate_proj.weight"] = torch.randn(I, H, generator=g)
        s[b + "up_proj.weight"] = torch.randn(I, H, generator=g)
        s[b + "down_proj.weight"] = torch.randn(H, I, generator=g)
    return s


@pytest.mark.parametrize("mutate, match", [
    (lambda s: s.pop("model.layers.0.mlp.experts.4.up_proj.weight"), r"expert 4: missing \['up_proj'\]"),
    (lambda s: [s.pop(k) for k in list(s) if ".experts.5." in k], "router has 6 experts"),
    (lambda s: s.__setitem__("model.layers.0.mlp.experts.6.gate_proj.weight", torch.zeros(I, H)),
     "router has 6 experts"),
    (lambda s: s.__setitem__("model.layers.0.mlp.experts.2.down_proj.weight", torch.zeros(I, H)),
     "expert 2: down"),
    (lambda s: s.__setitem__("model.layers.0.mlp.experts.1.gate_proj.weight", torch.zeros(I, H + 1)),
     "expert 1: gate"),
    (lambda s: s.__setitem__("model.layers.0.mlp.shared_expert.gate_proj.weight", torch.zeros(I, H)),
     "unsupported MoE key"),
    (lambda s: s.pop("model.layers.0.mlp.gate.weight"), "experts without a router"),
    (lambda s: s.__setitem__("model.layers.1.mlp.gate.weight", torch.zeros(E, H)), "router without experts"),
])
def test_malformed_checkpoints_raise(mutate, match):
    s = _state()
    mutate(s)
    with pytest.raises(AssertionError, match=match):
        pack_moe_state(s)


def test_ragged_intermediate_size_raises():
    s = _state()
    b = "model.layers.0.mlp.experts.3."
    s[b + "gate_proj.weight"] = torch.zeros(I + 8, H)
    s[b + "up_proj.weight"] = torch.zeros(I + 8, H)
    s[b + "down_proj.weight"] = torch.zeros(H, I + 8)
    with pytest.raises(AssertionError, match="intermediate size"):
        pack_moe_state(s)


def test_model_shape_mismatch_and_missing_files_raise(tmp_path):
    save_file(_state(), str(tmp_path / "model.safetensors"))
    with pytest.raises(AssertionError, match="num_experts must match"):
        load_hf_moe_weights(_WrongE(), tmp_path)
    with pytest.raises(AssertionError, match="not in the model"):
        load_hf_moe_weights(torch.nn.Linear(2, 2), tmp_path)
    with pytest.raises(AssertionError, match="neither"):
        weight_files(tmp_path / "nothing")


def test_index_lists_every_shard(tmp_path):
    s = _state()
    keys = sorted(s)
    half = len(keys) // 2
    save_file({k: s[k] for k in keys[:half]}, str(tmp_path / "a.safetensors"))
    save_file({k: s[k] for k in keys[half:]}, str(tmp_path / "b.safetensors"))
    wm = {k: ("a.safetensors" if i < half else "b.safetensors") for i, k in enumerate(keys)}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    got = read_state(tmp_path)
    assert set(got) == set(s) and all(torch.equal(got[k], s[k]) for k in s)


class _WrongE(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.blocks = torch.nn.ModuleList([torch.nn.Module()])
        self.blocks[0].ffn = Qwen3MoeSparseMLP(H, I, E + 2, K, True)
