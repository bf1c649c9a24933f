"""GPU parity of reax_rarn (reduce-add RMSNorm, libreax_howu/reax_rarn_final.cu) through the C ABI: h_out and out
bit-identical to the CPU oracle (which follows the reference's rounding order, with r in double precision like the
kernel), over partial counts 2..8, serial and plain partial sums, padded partial strides, ragged row counts, the
4-byte-aligned form and the reference's return codes."""
import numpy as np
import pytest

import pyoracle
import rarn_cases as RC
from reax_fmha import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

D = RC.D


def _say(msg):
    print(f"[gpu-rarn] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _to_dev(bits, offset=0):
    """bf16 bits on the device, starting `offset` elements into a fresh allocation (offset 2: only 4-byte aligned)."""
    buf = torch.zeros(bits.size + offset + 8, dtype=torch.bfloat16, device="cuda")
    t = buf[offset: offset + bits.size]
    t.copy_(W.bits_to_torch(bits.reshape(-1), "cuda"))
    return t


CASES = [  # n, S, serial, pad (elements between partials beyond n*D), offset (elements)
    (1, 2, 0, 0, 0),
    (7, 3, 1, 8, 0),
    (16, 5, 0, 0, 0),
    (33, 8, 1, 16, 0),
    (1000, 4, 0, 0, 0),
    (17, 6, 0, 0, 0),
    (9, 3, 0, 2, 2),   # 4-byte-aligned buffers and an odd pad: the 2-column-per-lane form
    (20, 7, 1, 6, 2),
]


@pytest.mark.parametrize("n,S,serial,pad,offset", CASES)
def test_rarn_matches_oracle(n, S, serial, pad, offset):
    from reax_fmha import ops

    _say(f"n={n} S={S} serial={serial} pad={pad} offset={offset}")
    eps, factor = 1e-6, 1.0 / D
    part, ps, res, w = RC.make_inputs(n, S, 1000 + n + S, pad=pad)
    code, h_ref, o_ref, _ = pyoracle.rarn(part, S, serial, ps, res, w, n, eps=eps, factor=factor)
    assert code == 0
    dpart, dres, dw = _to_dev(part, offset), _to_dev(res, offset), _to_dev(w, offset)
    h_out = _to_dev(np.zeros(n * D, np.uint16), offset).view(n, D)
    out = _to_dev(np.zeros(n * D, np.uint16), offset).view(n, D)
    ops.rarn(dpart, S, serial, ps, dres, dw, n, eps=eps, factor=factor, h_out=h_out, out=out)
    torch.cuda.synchronize()
    hg, og = W.torch_to_bits(h_out).reshape(n, D), W.torch_to_bits(out).reshape(n, D)
    bad_h = int((hg != h_ref).sum())
    bad_o = int((og != o_ref).sum())
    assert bad_h == 0, f"h_out differs from the oracle at {bad_h} elements"
    assert bad_o == 0, f"out differs from the oracle at {bad_o} elements"


def test_rarn_return_codes():
    from reax_fmha import abi

    L = abi.howu()
    part, ps, res, w = RC.make_inputs(2, 3, 5)
    dpart, dres, dw = _to_dev(part), _to_dev(res), _to_dev(w)
    h = torch.zeros((2, D), dtype=torch.bfloat16, device="cuda")
    o = torch.zeros((2, D), dtype=torch.bfloat16, device="cuda")
    args = lambda S, n, d: (dpart.data_ptr(), S, 0, ps, dres.data_ptr(), dw.data_ptr(), h.data_ptr(), o.data_ptr(),
                            n, d, 1e-6, 1.0 / D, None)
    assert L.reax_rarn(*args(3, 0, D)) == 0
    assert L.reax_rarn(*args(3, 2, 2048)) == -1
    assert L.reax_rarn(*args(9, 2, D)) == -2
    assert L.reax_rarn(*args(1, 2, D)) == -2
    torch.cuda.synchronize()
    assert not h.any() and not o.any(), "a rejected call wrote its outputs"
