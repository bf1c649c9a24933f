"""GPU parity of reax_conv_l2 / reax_conv_v (causal 4-tap conv + SiLU + L2 norm, libreax_howu/reax_conv_v2.cu)
through the C ABI: q, k and v bit-identical to the CPU oracle (the reference's rounding order, with 1 + exp(-y)
and 1/sqrt evaluated in double precision like the kernel), over rep 1 and 2, skip_v, sequences with and without
cached positions, token counts that do not fill a workgroup, the values-only entry point and the return codes."""
import numpy as np
import pytest

import conv_cases as CC
import pyoracle
from reax_fmha import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SENT = 0x7FBF  # a bf16 NaN pattern: outputs a call must not touch keep it


def _say(msg):
    print(f"[gpu-conv] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _dev_inputs(a):
    qkv = W.bits_to_torch(a["qkv"], "cuda")
    cache = W.bits_to_torch(a["cache"], "cuda")
    meta = torch.from_numpy(a["meta"]).cuda()
    w = W.bits_to_torch(a["w"], "cuda")
    return qkv, cache, meta, w


def _sent(shape):
    return W.bits_to_torch(np.full(shape, SENT, dtype=np.uint16), "cuda")


CASES = [  # seqs, KD, VD, rep, skip_v, RT
    (CC.SEQS, 128, 256, 1, 0, 16),
    ([(0, 40), (5, 33), (2, 1)], 256, 512, 2, 0, 8),
    ([(3, 17), (0, 2)], 256, 256, 1, 1, 32),
    ([(1, 64), (9, 64), (0, 3)], 128, 128, 2, 1, 16),
]


@pytest.mark.parametrize("seqs,KD,VD,rep,skip_v,RT", CASES)
def test_conv_l2_matches_oracle(seqs, KD, VD, rep, skip_v, RT):
    from reax_fmha import ops

    a = CC.make_inputs(seqs, KD, VD, 700 + KD + VD + rep)
    Tf = a["Tf"]
    _say(f"Tf={Tf} KD={KD} VD={VD} rep={rep} skip_v={skip_v} RT={RT}")
    eps = 1e-6
    q_ref, k_ref, v_ref, _ = CC.run(a, rep=rep, skip_v=skip_v, eps=eps)
    qkv, cache, meta, w = _dev_inputs(a)
    REP = 1 if rep == 1 else 2
    q, k, v = _sent((Tf, REP * KD)), _sent((Tf, REP * KD)), _sent((Tf, VD))
    ops.conv_l2(qkv, cache, meta, w, Tf=Tf, KD=KD, VD=VD, eps=eps, rep=rep, skip_v=skip_v, RT=RT, q=q, k=k, v=v)
    torch.cuda.synchronize()
    for name, got, ref in (("q", q, q_ref), ("k", k, k_ref)):
        g = W.torch_to_bits(got)
        bad = int((g != ref).sum())
        assert bad == 0, f"{name}: {bad} elements differ from the oracle"
    gv = W.torch_to_bits(v)
    if skip_v:
        assert (gv == SENT).all(), "skip_v: v was written"
    else:
        bad = int((gv != v_ref[:, :VD]).sum())
        assert bad == 0, f"v: {bad} elements differ from the oracle"


def test_conv_v_matches_oracle():
    from reax_fmha import ops

    a = CC.make_inputs([(0, 30), (4, 21)], 256, 384, 811)
    Tf, KD, VD = a["Tf"], a["KD"], a["VD"]
    _say(f"conv_v Tf={Tf} KD={KD} VD={VD}")
    _, _, v_ref, _ = pyoracle.conv(a["qkv"], a["SX"], a["cache"], a["C"], a["meta"], a["w"], Tf, KD=KD, VD=VD,
                                   u0=2 * KD // 128, units=VD // 128)
    qkv, cache, meta, w = _dev_inputs(a)
    v = ops.conv_v(qkv, cache, meta, w, Tf=Tf, KD=KD, VD=VD, v=_sent((Tf, VD)))
    torch.cuda.synchronize()
    bad = int((W.torch_to_bits(v) != v_ref).sum())
    assert bad == 0, f"v: {bad} elements differ from the oracle"


def test_conv_return_codes():
    from reax_fmha import abi

    L = abi.howu()
    a = CC.make_inputs(CC.SEQS, 128, 128, 5)
    qkv, cache, meta, w = _dev_inputs(a)
    out = _sent((a["Tf"], 256))
    base = lambda Tf, RT: (qkv.data_ptr(), a["SX"], cache.data_ptr(), a["C"], meta.data_ptr(), w.data_ptr(),
                           out.data_ptr(), out.data_ptr(), out.data_ptr(), Tf, 1e-6, 128, 128, 1, 0, RT, None)
    assert L.reax_conv_l2(*base(0, 16)) == 0
    assert L.reax_conv_l2(*base(a["Tf"], 12)) == -1
    assert L.reax_conv_v(qkv.data_ptr(), a["SX"], cache.data_ptr(), a["C"], meta.data_ptr(), w.data_ptr(),
                         out.data_ptr(), 0, 128, 128, None) == 0
    torch.cuda.synchronize()
    assert (W.torch_to_bits(out) == SENT).all(), "a rejected call wrote its outputs"
