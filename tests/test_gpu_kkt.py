"""GPU parity of reax_kkt (Gated-DeltaNet chunk solve, libreax_howu/reax_kkt.cu) through the C ABI against the
double-precision CPU oracle: every written entry within one bf16 ulp relative plus 1e-4 absolute (the kernel works
in fp32: entries that come out small by cancellation carry the fp32 rounding of their larger terms), entries outside the lower block triangle untouched, over varlen sequences with partial chunks,
several key heads, and the return codes. The reference itself agrees with the oracle only to its bf16 / tf32
tensor-core accuracy, so parity with it is tolerance-based."""
import numpy as np
import pytest

import kkt_cases as KC
from reax_fmha import workloads as W
from rarn_cases import bf16_to_f32

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _say(msg):
    print(f"[gpu-kkt] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _dev(a):
    return (W.bits_to_torch(a["k"], "cuda"), torch.from_numpy(a["g"]).cuda(), W.bits_to_torch(a["beta"], "cuda"),
            torch.from_numpy(a["cu"]).cuda(), torch.from_numpy(a["cidx"]).cuda())


@pytest.mark.parametrize("lens,H,seed", [([64], 1, 10), ([130, 64, 45], 2, 11), ([1, 2, 63, 65, 200], 4, 12),
                                          ([512, 300], 8, 13), ([4096, 4000, 130], 8, 15)])
def test_kkt_matches_oracle(lens, H, seed):
    # the last case has 130 chunks x 8 key heads = 1040 items, more than the persistent grid's KKT_WG_PER_CU (3)
    # workgroups on each of 256 CUs: workgroups run a second item (the prefetched next item, LDS reused)
    from reax_fmha import ops

    a = KC.make_inputs(lens, H, seed)
    _say(f"lens={lens} H={H} NT={a['NT']}")
    code, A_ref = KC.run(a)
    assert code == 0
    k, g, beta, cu, cidx = _dev(a)
    A = W.bits_to_torch(np.full((a["T"], a["HV"], 64), KC.SENT, np.uint16), "cuda")
    ops.kkt(k, g, beta, cu, cidx, NT=a["NT"], H=H, HV=a["HV"], A=A)
    torch.cuda.synchronize()
    Ag = W.torch_to_bits(A).reshape(a["T"], a["HV"], 64)
    m = np.broadcast_to(KC.written_mask(a)[:, None, :], Ag.shape)
    assert (Ag[~m] == KC.SENT).all(), "wrote outside the lower block triangle"
    got, want = bf16_to_f32(Ag[m]).astype(np.float64), bf16_to_f32(A_ref[m]).astype(np.float64)
    bad = np.abs(got - want) > np.abs(want) * 2.0 ** -7 + 1e-4  # one bf16 ulp is up to 2^-7 of the value
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} entries off by more than a bf16 ulp (max diff " \
                          f"{np.abs(got - want).max():.3g})"
    _say(f"bit-identical entries: {float((Ag[m] == A_ref[m]).mean()):.5f}")


def test_kkt_return_codes():
    from reax_fmha import abi

    L = abi.howu()
    a = KC.make_inputs([10], 1, 14)
    k, g, beta, cu, cidx = _dev(a)
    A = W.bits_to_torch(np.full((a["T"], 2, 64), KC.SENT, np.uint16), "cuda")
    args = lambda NT, H, HV: (k.data_ptr(), g.data_ptr(), beta.data_ptr(), A.data_ptr(), cu.data_ptr(),
                              cidx.data_ptr(), NT, H, HV, None)
    assert L.reax_kkt(*args(1, 1, 3)) == -1
    assert L.reax_kkt(*args(0, 1, 2)) == 9  # hipErrorInvalidConfiguration: empty grid
    torch.cuda.synchronize()
    assert (W.torch_to_bits(A) == KC.SENT).all(), "a rejected call wrote its output"
