"""GPU parity of the block-score and tier-label kernels: bit-exact against
the oracle's fixed-order reductions and its restatement of the reference's
policy (enforce_budget / enforce_tiered_budget, tierkv_policy.py:1391-1477,
itself checked against Python's stable ``sorted``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import policy as opolicy
from paged_tierkv_amd import kernels, workloads as W

pytestmark = pytest.mark.gpu


def _bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return x.view(np.uint32)


def test_c2b_block_mass_full_size_bit_exact(device):
    probs = W.config2b()
    print("[scores] C2(b) block mass [32, 32, 4096] -> [32, 256]", flush=True)
    got = kernels.block_mass_from_probs(probs.to(device), 16).cpu().numpy()
    exp = opolicy.block_mass_from_probs(probs.numpy(), 16)
    assert np.array_equal(_bits(got), _bits(exp))
    # the same quantity as the reference's mean-based scores, to fp32 rounding
    ref = probs.double().sum(dim=1).view(32, 256, 16).sum(-1) / 32 / 16
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-5, atol=1e-9)


def test_block_mass_with_lengths_bit_exact(device):
    g = torch.Generator().manual_seed(2)
    probs = torch.softmax(torch.randn((3, 5, 64 * 8), generator=g) * 2, dim=-1)
    for bs in (2, 4, 8, 16, 32, 64):
        nblk = probs.shape[-1] // bs
        lens = torch.randint(0, bs + 1, (3, nblk), generator=g, dtype=torch.int32)
        got = kernels.block_mass_from_probs(probs.to(device), bs, lens).cpu().numpy()
        exp = opolicy.block_mass_from_probs(probs.numpy(), bs, lens.numpy())
        assert np.array_equal(_bits(got), _bits(exp)), f"bs={bs}"


@pytest.mark.parametrize("shape", [(2, 40, 336, 16), (3, 71, 80, 4), (1, 1, 4, 4), (2, 33, 1024, 64),
                                   (2, 32, 832, 8), (1, 96, 512, 32)])
def test_block_mass_head_rounds_and_ragged_tiles_bit_exact(device, shape):
    # heads beyond one 32-head LDS round, token counts that leave a partial
    # 256-token workgroup, and the 4-byte-aligned (scalar) path
    b, h, t, bs = shape
    g = torch.Generator().manual_seed(sum(shape))
    probs = torch.softmax(torch.randn((b, h, t), generator=g) * 2, dim=-1)
    nblk = t // bs
    lens = torch.randint(0, bs + 1, (b, nblk), generator=g, dtype=torch.int32)
    print(f"[scores] block mass shape={shape}", flush=True)
    for ln in (None, lens):
        exp = opolicy.block_mass_from_probs(probs.numpy(), bs, None if ln is None else ln.numpy())
        got = kernels.block_mass_from_probs(probs.to(device), bs, ln).cpu().numpy()
        assert np.array_equal(_bits(got), _bits(exp)), f"aligned, lengths={ln is not None}"
        flat = torch.empty(probs.numel() + 1, device=device)
        un = flat[1:].view(b, h, t)
        un.copy_(probs.to(device))
        assert un.data_ptr() % 16 != 0
        got = kernels.block_mass_from_probs(un, bs, ln).cpu().numpy()
        assert np.array_equal(_bits(got), _bits(exp)), f"unaligned, lengths={ln is not None}"


def test_labels_at_the_block_limit(device):
    rng = np.random.default_rng(9)
    n = 8192
    scores = rng.integers(0, 50, (2, n)).astype(np.float32) / 7      # ties across passes
    cur = rng.integers(0, 3, (2, n)).astype(np.int32)
    print(f"[scores] labels n={n}", flush=True)
    exp = opolicy.tier_labels(scores, cur, 300, 2000, "hot_warm_cold")
    got = kernels.tier_labels(torch.from_numpy(scores).to(device), torch.from_numpy(cur).to(device), 300, 2000,
                              "hot_warm_cold").cpu().numpy()
    assert np.array_equal(got, exp)
    with pytest.raises(RuntimeError, match="too many blocks"):
        kernels.tier_labels(torch.zeros((1, n + 1), device=device), torch.zeros((1, n + 1), dtype=torch.int32,
                                                                                 device=device), 3, 3)


def test_c2b_labels_bit_exact(device):
    probs = W.config2b()
    mass = opolicy.block_mass_from_probs(probs.numpy(), 16)
    cur = np.zeros((32, 256), np.int32)
    exp = opolicy.tier_labels(mass, cur, W.C2B_HOT_BUDGET, W.C2B_WARM_BUDGET, "hot_warm_cold")
    got = kernels.tier_labels(torch.from_numpy(mass).to(device), torch.from_numpy(cur).to(device),
                              W.C2B_HOT_BUDGET, W.C2B_WARM_BUDGET, "hot_warm_cold").cpu().numpy()
    assert np.array_equal(got, exp)
    counts = [(int((r == 0).sum()), int((r == 1).sum()), int((r == 2).sum())) for r in got]
    assert set(counts) == {(26, 153, 77)}
    assert (got[:, 0] == 0).all() and (got[:, 255] == 0).all()


def test_reference_known_answer_labels(device):
    # main.py:375-389: block means [0.4, 0.9, 0.1, 0.2], hot_budget 3 -> [0, 0, 1, 0]
    scores = torch.tensor([[0.4, 0.9, 0.1, 0.2]], device=device)
    cur = torch.zeros((1, 4), dtype=torch.int32, device=device)
    got = kernels.tier_labels(scores, cur, 3, 0, "hot_warm", demoted_state=1)
    assert got.cpu().tolist() == [[0, 0, 1, 0]]


@pytest.mark.parametrize("mode", ["hot_warm", "hot_warm_cold", "hot_only"])
def test_labels_random_ties_sticky_cold(device, mode):
    rng = np.random.default_rng(5)
    for n in (1, 2, 3, 5, 17, 256, 2048):
        b = 6
        scores = rng.integers(0, 4, (b, n)).astype(np.float32) * 0.25     # many exact ties
        scores[1] = rng.standard_normal(n).astype(np.float32)
        scores[2] = 0.0                                                 # all tied
        scores[3, : n // 2] = -0.0                                      # -0.0 ties with 0.0
        cur = rng.integers(0, 3, (b, n)).astype(np.int32)
        cur[4] = 0
        hot, warm = int(rng.integers(0, n + 3)), int(rng.integers(0, n + 3))
        for demoted in (1, 2):
            exp = opolicy.tier_labels(scores, cur, hot, warm, mode, demoted_state=demoted)
            got = kernels.tier_labels(torch.from_numpy(scores).to(device), torch.from_numpy(cur).to(device),
                                      hot, warm, mode, demoted_state=demoted).cpu().numpy()
            assert np.array_equal(got, exp), f"mode={mode} n={n} hot={hot} warm={warm} demoted={demoted}"


def test_scores_from_sums_bit_exact(device):
    g = torch.Generator().manual_seed(8)
    sums = torch.rand((3, 32, 300), generator=g)
    lens = torch.randint(0, 17, (3, 300), generator=g, dtype=torch.int32)
    got = kernels.block_scores_from_sums(sums.to(device), lens.to(device), 256).cpu().numpy()
    exp = opolicy.block_mass_from_sums(sums.numpy(), lens.numpy(), 256)
    assert np.array_equal(_bits(got), _bits(exp))
    one = kernels.block_scores_from_sums(sums[0].to(device), lens[0].to(device), 10).cpu().numpy()
    assert np.array_equal(_bits(one), _bits(exp[0, :10]))
