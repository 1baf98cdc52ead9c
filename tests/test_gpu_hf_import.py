"""GPU: the HIP block on expert weights imported from a hub-layout checkpoint.

The checkpoint is written by transformers' own ``save_pretrained`` (one tensor
per expert and projection, the layout pluggy's importer reads,
pluggy/models/hf_import.py:72-99), loaded with ``load_hf_moe_weights`` into
the drop-in blocks on the GPU (fp32 masters), and run forward and backward on
the HIP kernels. The output is compared with transformers' own
``Qwen3MoeSparseMoeBlock`` and with the oracle's block on the same weights
(fp32, CPU), and every gradient with fp64 truth given the kernels' routing,
at the fp32 bar (rel-L2 <= 1e-4, max-abs <= 1e-4 of the largest magnitude).
"""

from __future__ import annotations

import os

import pytest
import torch

from oracle import moe_oracle as O
from tests._gpu_helpers import DEV, MAX_ABS_FRAC, check_close, gen, ref_layer_fp64, rel, say

pytestmark = pytest.mark.gpu

H, I, E, K, L = 256, 128, 16, 4, 2  # the kernels' multiples of 8


class _Blocks(torch.nn.Module):
    """Stand-in for the reference model's ``blocks`` list (qwen3_moe.py:371) holding drop-in FFNs."""

    class _Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            import pluggy_amd

            self.ffn = pluggy_amd.Qwen3MoeSparseMLP(H, I, E, K, True)

    def __init__(self):
        super().__init__()
        self.blocks = torch.nn.ModuleList(self._Block() for _ in range(L))


def test_hub_checkpoint_runs_on_the_hip_block(tmp_path):
    os.environ.setdefault("HF_HUB_OFFLINE", "1")
    transformers = pytest.importorskip("transformers")
    from pluggy_amd.hf_moe import load_hf_moe_weights

    cfg = transformers.Qwen3MoeConfig(
        vocab_size=32, hidden_size=H, intermediate_size=64, moe_intermediate_size=I, num_hidden_layers=L,
        num_attention_heads=2, num_key_value_heads=1, head_dim=8, num_experts=E, num_experts_per_tok=K,
        norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[], tie_word_embeddings=False)
    torch.manual_seed(0)
    hf = transformers.Qwen3MoeForCausalLM(cfg)
    g = gen(61)
    with torch.no_grad():
        for p in hf.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    hf.save_pretrained(tmp_path)
    model = _Blocks().to(DEV)
    n, _rest = load_hf_moe_weights(model, tmp_path)
    assert n == 3 * L
    f32 = torch.float32
    for layer in range(L):
        say(f"hub checkpoint layer {layer}: H={H} I={I} E={E} K={K} on the HIP block")
        ffn = model.blocks[layer].ffn
        assert ffn.experts.gate_up_proj.is_cuda and ffn.experts.gate_up_proj.dtype == f32
        x = torch.randn(2, 64, H, generator=g)
        gout = torch.randn(2 * 64, H, generator=g)
        xg = x.to(DEV).requires_grad_(True)
        out = ffn(xg)
        out.reshape(-1, H).backward(gout.to(DEV))
        torch.cuda.synchronize()
        logits = ffn.last_router_logits.detach().cpu()
        Wr = ffn.router.weight.detach().cpu()
        Wgu = ffn.experts.gate_up_proj.detach().cpu()
        Wdn = ffn.experts.down_proj.detach().cpu()
        with torch.no_grad():
            want_hf = hf.model.layers[layer].mlp(x)
            want_hf = want_hf[0] if isinstance(want_hf, tuple) else want_hf
            want_oracle, logits_o = O.sparse_mlp_forward(x, Wr, Wgu, Wdn, K, True)
        assert rel(logits, logits_o) < 1e-5
        idx = torch.from_numpy(O.select_topk(logits, K))
        assert torch.equal(idx, torch.from_numpy(O.select_topk(logits_o, K))), "routing differs from the CPU's"
        r_hf, r_o = rel(out.detach(), want_hf), rel(out.detach(), want_oracle)
        say(f"  out vs transformers' block rel={r_hf:.2e}, vs the oracle's block rel={r_o:.2e}")
        assert r_hf < 1e-4 and r_o < 1e-4
        ref = ref_layer_fp64(x.reshape(-1, H), Wr, Wgu, Wdn, idx, logits, True, gout=gout)
        frac = MAX_ABS_FRAC[f32]
        check_close("out", out.reshape(-1, H), ref["out"], 1e-4, frac)
        check_close("dx", xg.grad.reshape(-1, H), ref["dx"], 1e-4, frac)
        check_close("d router.weight", ffn.router.weight.grad, ref["dWr"], 1e-4, frac)
        check_close("d gate_up_proj", ffn.experts.gate_up_proj.grad, ref["dWgu"], 1e-4, frac)
        check_close("d down_proj", ffn.experts.down_proj.grad, ref["dWdn"], 1e-4, frac)
