"""GPU: reax_fmha_splitkv_noalloc, the split-KV entry point that allocates nothing (its partials live in the
library's static per-GPU scratch), against reax_fmha_splitkv with a caller workspace. Both run the same kernels,
so O and LSE must agree bit for bit: on two calls in a row, the second with a smaller input (its partials land on
a prefix of what the first call left in the scratch), and on a third call at the first shape again."""
import numpy as np
import pytest

import fmha_cases as FC
from reax_fmha import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _say(msg):
    print(f"[no-alloc] {msg}", flush=True)


CASES = [
    # config 4's shape (B 16, 8 KV heads, G 4, 8192 keys, 16 splits: 4.2 MB of partials)
    (FC.Case("na_c4", B=16, S=1, N=8192, Hq=32, Hkv=8, D=128, mode="causal", seed=201), 16),
    # smaller: 3 sequences, 2 query tokens, 1000 keys, 5 splits
    (FC.Case("na_small", B=3, S=2, N=1000, Hq=8, Hkv=2, D=128, mode="causal", seed=202), 5),
    # head_dim 256 (the 4-wavefront SPLIT kernel) after the two above
    (FC.Case("na_d256", B=2, S=3, N=700, Hq=4, Hkv=2, D=256, mode="causal", seed=203), 4),
]


def test_noalloc_matches_workspace_entry():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from reax_fmha import ops

    for i, (c, n) in enumerate(CASES + CASES[:1]):
        _say(f"call {i}: {c.name} B{c.B} S{c.S} N{c.N} Hq{c.Hq} Hkv{c.Hkv} D{c.D} splits{n}")
        a = FC.build(c)
        q, k, v = (W.bits_to_torch(a[x], "cuda") for x in ("q", "k", "v"))
        qpos = torch.from_numpy(a["qpos"]).cuda()
        o_ws, l_ws = ops.attention_splitkv(q, k, v, qpos, scale=c.scale, num_splits=n)
        o = torch.full_like(q, float("nan"))
        lse = torch.full((c.B, c.Hq, c.S), float("nan"), dtype=torch.float32, device="cuda")
        ops.attention_splitkv_noalloc(q, k, v, qpos, scale=c.scale, num_splits=n, o=o, lse=lse)
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), o_ws.view(torch.int16)), f"{c.name}: O differs from the workspace call"
        assert torch.equal(lse, l_ws), f"{c.name}: LSE differs from the workspace call"
        if c.name == "na_small":
            ref_o, ref_lse = FC.oracle_ref(c, a)
            FC.check_tolerance(W.torch_to_bits(o), ref_o, lse.cpu().numpy(), ref_lse, where=c.name)


def test_noalloc_rejects_oversize():
    """A shape whose partials exceed the 8 MiB scratch returns hipErrorOutOfMemory (2) before any launch."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from reax_fmha import abi

    qpos = torch.zeros((64, 1), dtype=torch.int32, device="cuda")
    o = torch.zeros((64, 1, 32, 128), dtype=torch.bfloat16, device="cuda")
    # B 64 x 8 KV heads x 64 splits x 4 rows x 129 floats = 67.6 MB > 8 MiB
    rc = abi.howu().reax_fmha_splitkv_noalloc(
        o.data_ptr(), o.data_ptr(), o.data_ptr(), qpos.data_ptr(), 4, 1, o.data_ptr(), None, 0.088, 64, 8, 4, 8192,
        128, 64, *([0] * 18), torch.cuda.current_stream().cuda_stream)
    assert rc == 2
    assert (o == 0).all()
