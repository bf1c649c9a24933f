"""GPU parity of reax_howu / howu3_dense (Gated-DeltaNet chunked forward, libreax_howu/reax_howu.cu) through the C
ABI against the CPU oracle with the reference's bf16 rounding points and the same bf16 chunk-solve A: max error
within 2^-6 and mean error within 2^-10 of the output scale (the matrix products accumulate in fp32 in the matrix
cores' order, the oracle in double, so bf16 roundings of intermediates can differ by an ulp and carry through the
state), every token row written, over varlen sequences with partial chunks and GQA ratios 1-3, including grids
of 16+ workgroups, where the kernel groups a key head's value heads onto one XCD. The oracle itself
equals the token-by-token gated delta rule when its roundings are dropped (tests/test_howu_oracle.py)."""
import numpy as np
import pytest

import howu_cases as HC
from reax_fmha import workloads as W
from rarn_cases import bf16_to_f32

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _say(msg):
    print(f"[gpu-howu] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.mark.parametrize("lens,H,HV,dense,seed", [([64], 1, 2, False, 20), ([70, 130], 1, 2, False, 21),
                                                   ([5, 200, 64], 2, 4, False, 22), ([150, 1], 1, 3, False, 23),
                                                   ([300], 4, 8, True, 24),
                                                   ([70, 1, 130, 64, 5, 128, 33, 200], 1, 2, False, 25),
                                                   ([100, 64, 3, 190, 64, 1, 77, 128], 2, 4, True, 26)])
def test_howu_matches_oracle(lens, H, HV, dense, seed):
    from reax_fmha import ops

    a = HC.make_inputs(lens, H, HV, seed)
    _say(f"lens={lens} H={H} HV={HV} dense={dense}")
    A = HC.chunk_solve(a)
    if dense:  # howu3_dense reads every block of A: give it zeros above the diagonal blocks, as the skip form reads
        m = np.zeros((a["T"], 64), bool)
        for i, L in enumerate(a["lens"]):
            for t in range(L):
                m[a["cu"][i] + t, : 16 * ((t % 64) // 16 + 1)] = True
        A = np.where(m[:, None, :], A, 0).astype(np.uint16)
    ref = HC.run(a, A=A)
    d = lambda x: W.bits_to_torch(x, "cuda")
    o = d(np.full((a["T"], HV, 128), HC.SENT, np.uint16))
    ops.howu(d(a["q"]), d(a["k"]), d(a["v"]), d(a["beta"]), d(A), torch.from_numpy(a["g"]).cuda(),
             torch.from_numpy(a["cu"]).cuda(), N=len(lens), H=H, HV=HV, scale=a["scale"], o=o, dense=dense)
    torch.cuda.synchronize()
    ob = W.torch_to_bits(o).reshape(a["T"], HV, 128)
    assert (ob != HC.SENT).all(), "a token row left unwritten"
    got, want = bf16_to_f32(ob).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    scale = np.abs(want).max()
    err = np.abs(got - want)
    _say(f"max err {err.max() / scale:.3g}, mean err {err.mean() / scale:.3g} of the output scale {scale:.3g}")
    assert err.max() <= scale * 2.0 ** -6, f"max error {err.max() / scale:.3g} of the output scale"
    assert err.mean() <= scale * 2.0 ** -10, f"mean error {err.mean() / scale:.3g} of the output scale"


@pytest.mark.parametrize("lens,H,HV,seed", [([70, 130], 1, 2, 30), ([5, 64, 100], 2, 4, 31)])
def test_howu_norm_matches_oracle(lens, H, HV, seed):
    """reax_howu_norm: the gated-RMSNorm epilogue rows (through f2s, some tokens dropped) against the epilogue of
    the oracle's o, same tolerance; rows no token addresses stay untouched."""
    from reax_fmha import ops

    a = HC.make_inputs(lens, H, HV, seed)
    n = HC.make_norm_inputs(a, seed + 100)
    _say(f"norm lens={lens} H={H} HV={HV}")
    A = HC.chunk_solve(a)
    ref = HC.norm_epilogue(HC.run(a, A=A), a, n)
    d = lambda x: W.bits_to_torch(x, "cuda")
    out = d(np.full((a["T"], HV, 128), HC.SENT, np.uint16))
    ops.howu_norm(d(a["q"]), d(a["k"]), d(a["v"]), d(a["beta"]), d(A), torch.from_numpy(a["g"]).cuda(),
                  torch.from_numpy(a["cu"]).cuda(), torch.from_numpy(n["f2s"]).cuda(),
                  d(n["z"]).reshape(a["T"], HV * 128), d(n["nw"]), N=len(lens), H=H, HV=HV, scale=a["scale"],
                  eps=n["eps"], factor=n["factor"], out=out)
    torch.cuda.synchronize()
    ob = W.torch_to_bits(out).reshape(a["T"], HV, 128)
    written = ref != HC.SENT
    assert (ob[~written] == HC.SENT).all(), "wrote a row no token addresses"
    got, want = bf16_to_f32(ob[written]).astype(np.float64), bf16_to_f32(ref[written]).astype(np.float64)
    scale = np.abs(want).max()
    err = np.abs(got - want)
    _say(f"max err {err.max() / scale:.3g}, mean err {err.mean() / scale:.3g} of the output scale {scale:.3g}")
    assert err.max() <= scale * 2.0 ** -6, f"max error {err.max() / scale:.3g} of the output scale"
    assert err.mean() <= scale * 2.0 ** -10, f"mean error {err.mean() / scale:.3g} of the output scale"


def test_howu_return_codes():
    from reax_fmha import abi

    L = abi.howu()
    a = HC.make_inputs([10], 1, 2, 25)
    d = lambda x: W.bits_to_torch(x, "cuda")
    q, k, v, beta = d(a["q"]), d(a["k"]), d(a["v"]), d(a["beta"])
    A = d(np.zeros((a["T"], 2, 64), np.uint16))
    g, cu = torch.from_numpy(a["g"]).cuda(), torch.from_numpy(a["cu"]).cuda()
    o = d(np.full((a["T"], 2, 128), HC.SENT, np.uint16))
    args = lambda N, H, HV: (q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), A.data_ptr(), g.data_ptr(),
                             o.data_ptr(), cu.data_ptr(), 0.1, N, H, HV, None)
    assert L.reax_howu(*args(0, 1, 2)) == 9   # empty grid: hipErrorInvalidConfiguration
    assert L.reax_howu(*args(1, 3, 2)) == 1   # H does not divide HV: hipErrorInvalidValue
    torch.cuda.synchronize()
    assert (W.torch_to_bits(o) == HC.SENT).all(), "a rejected call wrote its output"
