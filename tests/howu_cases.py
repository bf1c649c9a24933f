"""Inputs and independent checks for the Gated-DeltaNet chunked forward (reax_howu, libreax_howu/reax_howu.cu).

The chunked form computes, per sequence and value head, the gated delta rule
    S <- 2^(d_t) S;  S <- S + beta_t k_t (v_t - S^T k_t)^T;  o_t = scale * S^T q_t       (S: 128 k x 128 v, S_0 = 0)
with g the chunk-local cumulative sum of the per-token log2 decays d_t. Pins:
  - pin_recurrence: the oracle with every bf16 rounding dropped and the exact (I + M)^-1 equals this token-by-token
    recurrence (numpy float64) to one bf16 ulp of the output scale, over varlen sequences with partial chunks and
    GQA (several value heads per key head): the whole chunk algebra (u, w, the intra-chunk causal term, the decays
    of the inter-chunk term, of vdec and of the carried state);
  - pin_faithful: with the reference's bf16 rounding points and the bf16 A from the chunk solve, the oracle stays
    within bf16-level distance of the recurrence (the rounding points do not change the function);
  - pin_rows: rows of every token written, nothing else.
"""
from __future__ import annotations

import numpy as np

import pyoracle
from rarn_cases import bf16_to_f32, f32_to_bf16

SENT = 0x7FBF


def make_inputs(lens, H, HV, seed):
    rng = np.random.default_rng(seed)
    T = int(sum(lens))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    qf = rng.standard_normal((T, H, 128)).astype(np.float32)
    kf = rng.standard_normal((T, H, 128)).astype(np.float32)
    qf /= np.linalg.norm(qf, axis=2, keepdims=True)
    kf /= np.linalg.norm(kf, axis=2, keepdims=True)
    v = f32_to_bf16(rng.standard_normal((T, HV, 128)).astype(np.float32))
    beta = f32_to_bf16((1.0 / (1.0 + np.exp(-rng.standard_normal((T, HV))))).astype(np.float32))
    d = -rng.uniform(0.0, 0.15, size=(T, HV))
    g = np.zeros((T, HV), np.float32)
    for i in range(len(lens)):
        for c0 in range(cu[i], cu[i + 1], 64):
            c1 = min(c0 + 64, cu[i + 1])
            g[c0:c1] = np.cumsum(d[c0:c1], axis=0).astype(np.float32)
    return dict(q=f32_to_bf16(qf), k=f32_to_bf16(kf), v=v, beta=beta, g=g, cu=cu, T=T, H=H, HV=HV, lens=list(lens),
                scale=float(np.float32(1.0 / np.sqrt(128.0))))


def chunk_solve(a):
    """bf16 A from the chunk-solve oracle (the input reax_howu takes)."""
    cidx = np.array([(i, c) for i, L in enumerate(a["lens"]) for c in range((L + 63) // 64)], dtype=np.int64)
    H, HV = a["H"], a["HV"]
    if HV == 2 * H:
        return pyoracle.kkt(a["k"], a["g"], a["beta"], a["cu"], cidx, NT=len(cidx), H=H, HV=HV)[1]
    # general GQA ratio: solve per value head with its key head repeated
    rep = HV // H
    A = np.zeros((a["T"], HV, 64), np.uint16)
    for hv in range(HV):
        ksel = np.ascontiguousarray(np.repeat(a["k"][:, hv // rep: hv // rep + 1], 2, axis=1))
        gsel = np.ascontiguousarray(np.repeat(a["g"][:, hv: hv + 1], 2, axis=1))
        bsel = np.ascontiguousarray(np.repeat(a["beta"][:, hv: hv + 1], 2, axis=1))
        _, Ah = pyoracle.kkt(ksel[:, :1], gsel, bsel, a["cu"], cidx, NT=len(cidx), H=1, HV=2)
        A[:, hv] = Ah[:, 0]
    return A


def recurrence(a):
    """Token-by-token gated delta rule in float64: o [T][HV][128]."""
    T, H, HV = a["T"], a["H"], a["HV"]
    rep = HV // H
    q, k = bf16_to_f32(a["q"]).astype(np.float64), bf16_to_f32(a["k"]).astype(np.float64)
    v, beta = bf16_to_f32(a["v"]).astype(np.float64), bf16_to_f32(a["beta"]).astype(np.float64)
    g = a["g"].astype(np.float64)
    o = np.zeros((T, HV, 128))
    for i in range(len(a["lens"])):
        s0, s1 = a["cu"][i], a["cu"][i + 1]
        for hv in range(HV):
            S = np.zeros((128, 128))
            for t in range(s0, s1):
                first = (t - s0) % 64 == 0
                dt = g[t, hv] if first else g[t, hv] - g[t - 1, hv]
                S *= 2.0 ** dt
                kt, vt = k[t, hv // rep], v[t, hv]
                S += beta[t, hv] * np.outer(kt, vt - S.T @ kt)
                o[t, hv] = a["scale"] * (S.T @ q[t, hv // rep])
    return o


def run(a, *, exact=False, A=None, mutant=0):
    o = np.full((a["T"], a["HV"], 128), SENT, np.uint16)
    return pyoracle.howu(a["q"], a["k"], a["v"], a["beta"], A, a["g"], a["cu"], N=len(a["lens"]), H=a["H"],
                         HV=a["HV"], scale=a["scale"], exact=exact, o=o, mutant=mutant)


def _close(o_bits, ref, rel):
    got = bf16_to_f32(o_bits).astype(np.float64)
    scale = np.abs(ref).max()
    err = np.abs(got - ref).max() / scale
    return err, err <= rel


def pin_recurrence(mutant=0):
    for lens, H, HV, seed in [([70, 130], 1, 2, 1), ([64, 5], 2, 4, 2), ([150], 1, 3, 3)]:
        a = make_inputs(lens, H, HV, seed)
        ref = recurrence(a)
        err, ok = _close(run(a, exact=True, mutant=mutant), ref, 2.0 ** -8)
        assert ok, f"exact chunked form != recurrence: max error {err:.3g} of the output scale (lens {lens})"


def pin_faithful(mutant=0):
    a = make_inputs([130, 40], 1, 2, 4)
    ref = recurrence(a)
    err, ok = _close(run(a, A=chunk_solve(a), mutant=mutant), ref, 2.0 ** -4)
    assert ok, f"faithful chunked form off the recurrence by {err:.3g} of the output scale"


def pin_rows(mutant=0):
    a = make_inputs([3, 64, 1], 1, 2, 5)
    o = run(a, A=chunk_solve(a), mutant=mutant)
    assert (o != SENT).all(), "a token row left unwritten"


ALL_PINS = [pin_recurrence, pin_faithful, pin_rows]


# ------------------------------------------------------------------------------ gated-norm epilogue (reax_howu_norm)

def make_norm_inputs(a, seed, *, drop=0.2):
    """f2s (token -> output row, some tokens -1), gate z [rows][HV][128] bf16 (row stride HV*128), norm weight [128]."""
    rng = np.random.default_rng(seed)
    T, HV = a["T"], a["HV"]
    rows = rng.permutation(T).astype(np.int32)
    rows[rng.random(T) < drop] = -1
    z = f32_to_bf16((rng.standard_normal((T, HV, 128)) * 2.0).astype(np.float32))
    nw = f32_to_bf16((1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    return dict(f2s=rows, z=z, ZS=HV * 128, nw=nw, eps=1e-6, factor=1.0 / 128)


def norm_epilogue(o_bits, a, n):
    """The gated-RMSNorm epilogue of reax_howu_norm (norm_v3:347-392) on the chunked forward's bf16 o, in numpy
    float32 with its rounding points: out [T][HV][128] bf16 bits, rows not addressed left at SENT."""
    T, HV = a["T"], a["HV"]
    f = np.float32
    out = np.full((T, HV, 128), SENT, np.uint16)
    x = bf16_to_f32(o_bits)                                   # [T][HV][128]
    sq = (x * x).astype(f).reshape(T, HV, 32, 4)
    p = (((sq[..., 0] + sq[..., 1]).astype(f) + sq[..., 2]).astype(f) + sq[..., 3]).astype(f)  # [T][HV][32]
    for d in (16, 8, 4, 2, 1):
        p = p.copy()
        p[..., :d] = (p[..., :d] + p[..., d:2 * d]).astype(f)
    tot = p[..., 0]
    rr = (1.0 / np.sqrt(((tot * f(n["factor"])).astype(f) + f(n["eps"])).astype(f).astype(np.float64))).astype(f)
    y = bf16_to_f32(f32_to_bf16((x * rr[..., None]).astype(f)))
    w = bf16_to_f32(n["nw"])
    y2 = bf16_to_f32(f32_to_bf16((w[None, None, :] * y).astype(f)))
    for t in range(T):
        R = n["f2s"][t]
        if R < 0:
            continue
        zz = bf16_to_f32(n["z"][R]).astype(np.float64)
        d1 = (1.0 + np.exp(-zz)).astype(f)
        sz = (bf16_to_f32(n["z"][R]) / d1).astype(f)
        out[R] = f32_to_bf16((y2[t] * sz).astype(f))
    return out


def pin_norm_formula(mutant=0):
    """The epilogue against the float64 gated RMSNorm y = w * o / sqrt(mean(o^2) + eps) * silu(z) to 2 bf16 ulps
    (the factor 1/128 makes sum * factor the mean)."""
    a = make_inputs([70, 30], 1, 2, 9)
    o = run(a, A=chunk_solve(a), mutant=mutant)
    n = make_norm_inputs(a, 10)
    out = norm_epilogue(o, a, n)
    x = bf16_to_f32(o).astype(np.float64)
    w = bf16_to_f32(n["nw"]).astype(np.float64)
    for t in range(a["T"]):
        R = n["f2s"][t]
        if R < 0:
            continue
        zz = bf16_to_f32(n["z"][R]).astype(np.float64)
        want = w * x[t] / np.sqrt((x[t] ** 2).mean(axis=1, keepdims=True) + n["eps"]) * (zz / (1 + np.exp(-zz)))
        got = bf16_to_f32(out[R]).astype(np.float64)
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -6 + 1e-6), f"norm epilogue off at token {t}"


ALL_PINS.append(pin_norm_formula)
