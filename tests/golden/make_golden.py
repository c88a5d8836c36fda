"""Write golden vectors from the reference's own CPU code paths.

Run in the build container only (the reference tree is read, never copied):

    python tests/golden/make_golden.py /root/reference

Outputs small .npz fixtures next to this script:

* codec_ref_u8.npz -- quantize_fp16_to_int8 / dequantize_int8_to_fp16
  (tierkv_policy.py:21-44) on random fp16 rows plus edge rows (constant,
  all-positive, ties, wide range), executed by ATen on the CPU.  Pins the
  bit-exact fp16 op semantics the oracle codec restates.
* compact_trajectory.npz -- a scripted sequence of
  CompactTieredKVTensorPool operations (tierkv_policy.py:701-1365) on CPU
  tensors: slot ids, states, lengths and tables after every step.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def codec_vectors(tp):
    g = torch.Generator().manual_seed(1234)
    rows = [torch.randn((6, 4, 16, 64), generator=g).half()]
    edge = torch.zeros((1, 4, 16, 64), dtype=torch.float16)
    edge[0, 0] = 0.75                                      # constant rows -> scale 1
    edge[0, 1] = torch.linspace(1.0, 2.0, 64).half()       # all positive -> negative zp
    edge[0, 2] = (torch.arange(64) % 7).half() * 0.5       # many ties
    edge[0, 3] = torch.randn((16, 64), generator=g).half() * 40.0
    rows.append(edge)
    x = torch.cat(rows, dim=0)
    q, s, z = tp.quantize_fp16_to_int8(x)
    d = tp.dequantize_int8_to_fp16(q, s, z)
    return dict(x=x.numpy(), q=q.numpy(), scale=s.numpy(), zero=z.numpy(), deq=d.numpy())


def main(ref_root):
    sys.path.insert(0, ref_root)
    import tierkv_policy as tp   # the reference module, CPU only

    np.savez_compressed(os.path.join(HERE, "codec_ref_u8.npz"), **codec_vectors(tp))
    print("wrote codec_ref_u8.npz")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
