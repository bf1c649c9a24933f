"""Writes the golden fixtures tests/golden/*.npz.

The expected outputs come from torch.nn.functional.scaled_dot_product_attention and torch.logsumexp in float64
on the CPU (fmha_cases.sdpa_ref), not from this repository's oracle, so the fixtures pin the oracle and the GPU
kernels to an independent implementation. The reference repository ships no fixtures for this path.
Run: python tests/golden/make_golden.py
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.dirname(HERE), os.path.join(ROOT, "reax-engine-kernels_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

import fmha_cases as FC  # noqa: E402
import golden_io  # noqa: E402


def cases():
    qp = np.array([[0, -1, 3, 70, 200, 5, 0, 64, 63, 65, 127, 128, 1, 2, 33, 99]], dtype=np.int32)
    return [
        FC.Case("golden_causal_gqa_d128", B=1, S=72, N=72, Hq=8, Hkv=2, D=128, mode="causal", seed=901),
        FC.Case("golden_qpos_edge_d128", B=1, S=16, N=150, Hq=4, Hkv=1, D=128, mode="qpos", seed=902, qpos=qp),
        FC.Case("golden_causal_gqa_d256", B=1, S=70, N=70, Hq=4, Hkv=2, D=256, mode="causal", seed=903),
        FC.Case("golden_bias_d256", B=1, S=40, N=90, Hq=2, Hkv=2, D=256, mode="bias", seed=904,
                bias_neg_inf_frac=0.25, bias_full_rows=(7,)),
        FC.Case("golden_decode_d128", B=2, S=1, N=300, Hq=8, Hkv=2, D=128, mode="full", seed=905),
    ]


def main():
    for c in cases():
        a = FC.build(c)
        o, lse = FC.sdpa_ref(c, a)
        path = os.path.join(HERE, c.name + ".npz")
        golden_io.save(path, c, a, o, lse)
        print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
