"""Inputs and independent checks for the Gated-DeltaNet chunk solve (reax_kkt, libreax_howu/reax_kkt.cu).

A = (I + M)^-1 per 64-token chunk and value head, M[r][c] = (k_r . k_c) 2^(g[r] - g[c]) beta[r] for c < r. Pins:
  - pin_codes: HV != 2H returns -1 (kkt:265);
  - pin_identity: mutually orthogonal k rows make M = 0, so A is the identity on the written lower block triangle;
  - pin_two_rows: a 2-token sequence, A[1][0] = -(k_1 . k_0) 2^(g1 - g0) beta_1 worked out by hand, A[0][0] =
    A[1][1] = 1, A[0][1] = 0 (decay direction, which beta, the sign);
  - pin_inverse: (I + M) A = I to bf16 accuracy with M built in numpy from the formula, over varlen sequences with
    partial chunks (the whole inverse, the strictly-lower mask);
  - pin_layout: rows past a sequence's end and columns past a row's 16-column block are left untouched.
"""
from __future__ import annotations

import numpy as np

import pyoracle
from rarn_cases import bf16_to_f32, f32_to_bf16

SENT = 0x7FBF  # bf16 NaN: entries a call must not write


def make_inputs(lens, H, seed, *, orth=False):
    rng = np.random.default_rng(seed)
    HV = 2 * H
    T = int(sum(lens))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    if orth:
        kf = np.zeros((T, H, 128), np.float32)
        for t in range(T):
            kf[t, :, t % 128] = 1.0
    else:
        kf = rng.standard_normal((T, H, 128)).astype(np.float32)
        kf /= np.linalg.norm(kf, axis=2, keepdims=True)
    k = f32_to_bf16(kf)
    g = np.zeros((T, HV), np.float32)
    for i in range(len(lens)):
        s0, s1 = cu[i], cu[i + 1]
        g[s0:s1] = np.cumsum(-rng.uniform(0.0, 0.2, size=(s1 - s0, HV)), axis=0).astype(np.float32)
    beta = f32_to_bf16((1.0 / (1.0 + np.exp(-rng.standard_normal((T, HV))))).astype(np.float32))
    cidx = np.array([(i, c) for i, L in enumerate(lens) for c in range((L + 63) // 64)], dtype=np.int64)
    return dict(k=k, g=g, beta=beta, cu=cu, cidx=cidx, NT=len(cidx), H=H, HV=HV, T=T, lens=list(lens))


def run(a, mutant=0):
    A = np.full((a["T"], a["HV"], 64), SENT, dtype=np.uint16)
    code, A = pyoracle.kkt(a["k"], a["g"], a["beta"], a["cu"], a["cidx"], NT=a["NT"], H=a["H"], HV=a["HV"], A=A,
                           mutant=mutant)
    return code, A


def written_mask(a):
    """[T][64] True where reax_kkt writes (row r of its chunk: columns < 16 * (r // 16 + 1))."""
    m = np.zeros((a["T"], 64), bool)
    for i, L in enumerate(a["lens"]):
        for t in range(L):
            r = t % 64
            m[a["cu"][i] + t, : 16 * (r // 16 + 1)] = True
    return m


def m_numpy(a, hv, i, c0):
    """M of sequence i, chunk starting at token c0, value head hv, from the formula (float64)."""
    s0 = a["cu"][i] + c0
    n = min(64, a["lens"][i] - c0)
    kf = bf16_to_f32(a["k"][s0:s0 + n, hv // 2]).astype(np.float64)
    raw = kf @ kf.T
    gg = a["g"][s0:s0 + n, hv]
    dg = (gg[:, None] - gg[None, :]).astype(np.float32).astype(np.float64)
    bt = bf16_to_f32(a["beta"][s0:s0 + n, hv]).astype(np.float64)
    return np.tril(raw * np.exp2(dg) * bt[:, None], -1), n


def pin_codes(mutant=0):
    a = make_inputs([5], 1, 0)
    code, _ = pyoracle.kkt(a["k"], a["g"], a["beta"], a["cu"], a["cidx"], NT=1, H=1, HV=3, mutant=mutant)
    assert code == -1


def pin_identity(mutant=0):
    a = make_inputs([70, 20], 2, 1, orth=True)
    code, A = run(a, mutant)
    assert code == 0
    m = written_mask(a)
    for hv in range(a["HV"]):
        Af = bf16_to_f32(A[:, hv, :])
        for i, L in enumerate(a["lens"]):
            for t in range(L):
                row = a["cu"][i] + t
                want = np.zeros(64, np.float32)
                want[t % 64] = 1.0
                got = np.where(m[row], Af[row], 0.0)
                assert np.array_equal(got, np.where(m[row], want, 0.0)), f"identity broken at row {row}"


def pin_two_rows(mutant=0):
    a = make_inputs([2], 1, 2)
    code, A = run(a, mutant)
    assert code == 0
    kf = bf16_to_f32(a["k"][:, 0]).astype(np.float64)
    for hv in range(2):
        g0, g1 = a["g"][0, hv], a["g"][1, hv]
        b1 = float(bf16_to_f32(a["beta"][1:2, hv])[0])
        want10 = -(kf[1] @ kf[0]) * 2.0 ** float(np.float32(g1 - g0)) * b1
        Af = bf16_to_f32(A[:2, hv, :2]).astype(np.float64)
        assert Af[0, 0] == 1.0 and Af[1, 1] == 1.0 and Af[0, 1] == 0.0, f"unit lower triangle broken: {Af}"
        assert abs(Af[1, 0] - want10) <= abs(want10) * 2.0 ** -8, f"A[1][0] {Af[1, 0]} != {want10}"


def pin_inverse(mutant=0):
    a = make_inputs([130, 64, 45], 2, 3)
    code, A = run(a, mutant)
    assert code == 0
    for i, L in enumerate(a["lens"]):
        for c0 in range(0, L, 64):
            for hv in range(a["HV"]):
                M, n = m_numpy(a, hv, i, c0)
                s0 = a["cu"][i] + c0
                Ab = A[s0:s0 + n, hv, :n]
                Af = np.tril(bf16_to_f32(Ab).astype(np.float64))  # the written lower triangle (upper part is 0)
                res = (np.eye(n) + M) @ Af - np.eye(n)
                scale = (np.abs(np.eye(n) + M) @ np.abs(Af)).max()
                err = np.abs(res).max() / scale
                assert err < 2.0 ** -7, f"(I + M) A != I: relative residual {err:.3g} (seq {i}, chunk {c0}, hv {hv})"


def pin_layout(mutant=0):
    a = make_inputs([70, 9], 1, 4)
    code, A = run(a, mutant)
    assert code == 0
    m = written_mask(a)
    for hv in range(a["HV"]):
        assert (A[:, hv, :][~m] == SENT).all(), "wrote outside the lower block triangle"
        assert (A[:, hv, :][m] != SENT).all(), "left part of the lower block triangle unwritten"


ALL_PINS = [pin_codes, pin_identity, pin_two_rows, pin_inverse, pin_layout]
