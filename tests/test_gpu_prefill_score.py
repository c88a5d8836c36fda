"""GPU parity of the prefill block-score kernel (tierkv_prefill_block_mass)
against the float64 oracle (oracle.policy.prefill_block_mass): per-sequence
mean causal attention probability per block over heads and queries, the
quantity compute_block_scores (tierkv_policy.py:1380-1389) takes from the
eager prefill attention.  fp16 / bf16 inputs are exact in the oracle; the
kernel accumulates q . k in fp32 on MFMA and uses exp2f, so the result is
compared at 1e-4 relative.  Covers ragged prompt lengths (not multiples of
16 or 64), GQA groups 1 / 4 / 8, head_dim 64 / 128, block sizes 16 / 32,
HF's transposed projection layout, bf16, and agreement with the tier
engine's compute_block_scores on materialised weights."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.policy import prefill_block_mass as oracle_mass
from paged_tierkv_amd import kernels, tierkv_policy as tp

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,H,Hkv,T,D,bs,dtype", [
    (1, 32, 8, 130, 128, 16, torch.float16),
    (2, 8, 8, 77, 64, 16, torch.float16),
    (2, 16, 2, 200, 128, 32, torch.float16),
    (1, 32, 4, 64, 128, 16, torch.bfloat16),
    (3, 4, 1, 1, 64, 16, torch.float16),
    (1, 16, 4, 513, 128, 16, torch.float16),
    (1, 12, 2, 300, 128, 16, torch.float16),     # GQA group 6: the guarded 8-head variant
    (2, 4, 2, 97, 64, 32, torch.bfloat16),       # GQA group 2: the guarded 4-head variant
])
def test_prefill_block_mass_matches_oracle(device, B, H, Hkv, T, D, bs, dtype):
    print(f"[prefill] B={B} H={H} Hkv={Hkv} T={T} D={D} bs={bs} {dtype}", flush=True)
    g = torch.Generator().manual_seed(T * 7 + H)
    q = (torch.randn((B, H, T, D), generator=g) * 1.5).to(dtype)
    k = (torch.randn((B, Hkv, T, D), generator=g) * 1.5).to(dtype)
    scaling = D ** -0.5
    got = kernels.prefill_block_mass(q.to(device), k.to(device), bs, scaling).cpu().numpy()
    want = oracle_mass(q.float().numpy(), k.float().numpy(), scaling, bs)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-9)


def test_prefill_block_mass_hf_layout(device):
    """q / k as HF produces them: [B, T, H, D] storage viewed as [B, H, T, D]."""
    B, H, Hkv, T, D = 2, 32, 8, 150, 128
    g = torch.Generator().manual_seed(3)
    q = torch.randn((B, T, H, D), generator=g).half().to(device).transpose(1, 2)
    k = torch.randn((B, T, Hkv, D), generator=g).half().to(device).transpose(1, 2)
    got = kernels.prefill_block_mass(q, k, 16, D ** -0.5).cpu().numpy()
    want = oracle_mass(q.float().cpu().numpy(), k.float().cpu().numpy(), D ** -0.5, 16)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-9)


def test_prefill_block_mass_agrees_with_compute_block_scores(device):
    """One sequence: the kernel equals the tier engine's compute_block_scores
    on the materialised fp32 causal probabilities (block-mass kernel)."""
    H, Hkv, T, D = 8, 2, 96, 64
    g = torch.Generator().manual_seed(9)
    q = torch.randn((1, H, T, D), generator=g).half().to(device)
    k = torch.randn((1, Hkv, T, D), generator=g).half().to(device)
    kk = k.float().repeat_interleave(H // Hkv, dim=1)
    logits = (q.float() @ kk.transpose(2, 3).contiguous()) * D ** -0.5
    logits = logits.masked_fill(~torch.tril(torch.ones(T, T, dtype=torch.bool, device=device)), float("-inf"))
    probs = torch.softmax(logits, dim=-1)
    engine = tp.TierKVPolicyEngine(block_size=16, block_manager=None)
    ref = engine.compute_block_scores(probs)
    got = kernels.prefill_block_mass(q, k, 16, D ** -0.5)[0]
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-8)
