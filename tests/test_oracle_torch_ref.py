"""The torch-CPU restatements of the reference's eager decode (the timed CPU
baseline) against the NumPy oracle, on tiered cases of both WARM formats and
both COLD modes, and on all-HOT inputs against dense softmax attention."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decode as odecode
from oracle import torch_ref
from paged_tierkv_amd import workloads as W

from helpers import assert_close, oracle_warm


def _torch_inputs(case, warm):
    qk, qv, sk, zk, sv, zv = warm
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a))
    return (case.query, case.block_table, case.block_states, case.block_lengths, case.hot_k, case.hot_v,
            t(qk), t(qv), t(sk), t(zk), t(sv), t(zv), case.num_blocks, case.groups, case.scaling)


@pytest.mark.parametrize("fmt,cold", [("absmax_i8", "masked"), ("ref_u8", "zero_logit"),
                                      ("absmax_i8", "zero_logit"), ("ref_u8", "masked")])
@pytest.mark.parametrize("fn", ["eager_decode_looped", "vectorized_decode"])
def test_torch_ref_matches_oracle(fmt, cold, fn):
    gen = torch.Generator().manual_seed(3)
    lengths = torch.randint(1, 17, (3, 40), generator=gen)
    case = W.make_tiered_case("torch_ref", 3, 16, 4, 64, 40, 8, 20, seed=9, lengths=lengths, max_blocks=44)
    warm = oracle_warm(case, fmt)
    out = getattr(torch_ref, fn)(*_torch_inputs(case, warm), warm_format=fmt, cold_mode=cold)
    exp = odecode.decode_attention(case.query[:, :, 0].numpy(), case.block_table.numpy(), case.block_states.numpy(),
                                   case.block_lengths.numpy(), case.num_blocks, case.hot_k.numpy(),
                                   case.hot_v.numpy(), *warm, case.groups, case.scaling, warm_format=fmt,
                                   cold_mode=cold)
    assert out.shape == (3, 1, 16, 64) and out.dtype == torch.float16
    assert_close(out[:, 0].float().numpy(), exp, what=f"{fn} {fmt} {cold}")


def test_torch_ref_all_hot_is_dense_attention():
    case = W.make_tiered_case("torch_ref_hot", 2, 8, 2, 64, 12, 12, 0, seed=4)
    warm = oracle_warm(case, "absmax_i8")
    out = torch_ref.eager_decode_looped(*_torch_inputs(case, warm), warm_format="absmax_i8", cold_mode="masked")
    # Dense K/V in logical order from the HOT pool.
    for b in range(2):
        k = torch.stack([case.hot_k[int(case.block_table[b, i])] for i in range(12)], 1).float()
        v = torch.stack([case.hot_v[int(case.block_table[b, i])] for i in range(12)], 1).float()
        k = k.reshape(2, -1, 64).repeat_interleave(4, 0)
        v = v.reshape(2, -1, 64).repeat_interleave(4, 0)
        ln = case.block_lengths[b, :12].tolist()
        keep = torch.cat([torch.arange(16) < n for n in ln])
        q = case.query[b, :, 0].float()
        p = torch.softmax((torch.einsum("hd,htd->ht", q, k) * case.scaling).masked_fill(~keep, float("-inf")), -1)
        ref = torch.einsum("ht,htd->hd", p, v)
        torch.testing.assert_close(out[b, 0].float(), ref, atol=2e-3, rtol=1e-2)
