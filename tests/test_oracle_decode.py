"""Pins for the oracle decode (CPU): textbook attention on all-HOT inputs
(torch SDPA in fp32), closed-form COLD identities, GQA/MHA equivalence, the
reference's score normalisation, and the BASELINE ideal-byte figures."""

from __future__ import annotations

import numpy as np
import torch

from oracle import decode as D
from paged_tierkv_amd import workloads as W

from helpers import oracle_decode, oracle_warm


def _small(states, lengths=None, groups=2, kv=2, dim=32, seed=0):
    nb = len(states)
    case = W.make_tiered_case("t", 1, kv * groups, kv, dim, nb, nb, 0, seed=seed,
                              lengths=None if lengths is None else [lengths], max_blocks=nb + 2,
                              layout="dense", dense_pool_blocks=nb + 3)
    case.block_states[0, :nb] = torch.tensor(states, dtype=torch.int32)
    return case


def test_all_hot_equals_sdpa():
    case = _small([0, 0, 0], lengths=[16, 16, 7], groups=4, kv=2, dim=64, seed=1)
    warm = oracle_warm(case, "absmax_i8")
    out = oracle_decode(case, warm, "absmax_i8", "masked")[0]
    slots = case.block_table[0, :3].long()
    k = torch.cat([case.hot_k[s].float() for s in slots], dim=1)[:, :39]
    v = torch.cat([case.hot_v[s].float() for s in slots], dim=1)[:, :39]
    k = k.repeat_interleave(4, dim=0)
    v = v.repeat_interleave(4, dim=0)
    q = case.query[0].float()                       # [H, 1, D]
    ref = torch.nn.functional.scaled_dot_product_attention(q[None], k[None], v[None], scale=case.scaling)[0, :, 0]
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-5, rtol=1e-5)


def test_all_cold_zero_logit_is_exactly_zero():
    case = _small([2, 2], lengths=[16, 3])
    warm = oracle_warm(case, "ref_u8")
    out, sc = oracle_decode(case, warm, "ref_u8", "zero_logit", True)
    assert np.all(out == 0)
    np.testing.assert_allclose(sc[0, :, :2], np.tile([16 / 19, 3 / 19], (4, 1)), rtol=1e-12)


def test_masked_cold_equals_zero_length_block():
    case = _small([0, 2, 1], lengths=[16, 16, 16], seed=2)
    warm = oracle_warm(case, "absmax_i8")
    a = oracle_decode(case, warm, "absmax_i8", "masked")
    case.block_states[0, 1] = 0
    case.block_lengths[0, 1] = 0
    b = oracle_decode(case, warm, "absmax_i8", "masked")
    np.testing.assert_array_equal(a, b)


def test_zero_logit_cold_equals_zero_hot_block():
    case = _small([0, 2, 0], lengths=[16, 9, 16], seed=3)
    warm = oracle_warm(case, "ref_u8")
    a = oracle_decode(case, warm, "ref_u8", "zero_logit")
    slot = int(case.block_table[0, 1])
    case.hot_k[slot] = 0
    case.hot_v[slot] = 0
    case.block_states[0, 1] = 0
    b = oracle_decode(case, warm, "ref_u8", "zero_logit")
    np.testing.assert_allclose(a, b, atol=1e-15)


def test_gqa_group_one_is_per_head_mha():
    case = _small([0, 1, 0], groups=1, kv=4, dim=16, seed=4)
    warm = oracle_warm(case, "absmax_i8")
    full = oracle_decode(case, warm, "absmax_i8", "masked")[0]
    for h in range(4):
        sub = _small([0, 1, 0], groups=1, kv=4, dim=16, seed=4)
        sub.query = sub.query[:, h:h + 1]
        sub.num_heads = 1
        sub.kv_heads = 1
        sub.hot_k, sub.hot_v = sub.hot_k[:, h:h + 1], sub.hot_v[:, h:h + 1]
        w = tuple(None if a is None else a[:, h:h + 1] for a in warm)
        got = oracle_decode(sub, w, "absmax_i8", "masked")[0]
        np.testing.assert_allclose(got[0], full[h], rtol=1e-12)


def test_scores_normalised_per_head():
    case = W.config1()
    warm = oracle_warm(case, "ref_u8")
    _, sc = oracle_decode(case, warm, "ref_u8", "zero_logit", True)
    np.testing.assert_allclose(sc[0, :, :32].sum(-1), 1.0, rtol=1e-12)


def test_ideal_bytes_match_baseline_figures():
    c1 = W.config1()
    c3 = W.config3(with_data=False)
    c4 = W.config4(with_data=False)
    for case, want in ((c1, 271_232), (c3, 216_944_640), (c4, 147_986_944)):
        args = (case.block_states.numpy(), case.num_blocks, case.num_heads, case.kv_heads, case.head_dim)
        assert D.ideal_bytes(*args) == want
        assert W.ideal_bytes(*args) == want
