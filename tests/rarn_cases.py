"""Inputs and independent checks for the reduce-add RMSNorm (reax_rarn, libreax_howu/reax_rarn_final.cu).

The pins below fix what the oracle must compute without re-running its code path:
  - pin_codes: the reference's return codes (rarn_final.cu:100, 104);
  - pin_h_numpy: h = bf16(res + bf16(sum of partials)) with numpy float32 arithmetic, partials added in order, and
    the serial variant's per-add rounding (rarn_final.cu:47-55);
  - pin_h_rounding: hand-worked cases where the serial rounding and the rounding of d before the residual change
    the result (1 + 2^-8 + 2^-8 and the like, exact in bf16 arithmetic);
  - pin_rms_formula: out against the float64 RMSNorm h / sqrt(factor * sum(h^2) + eps) * (1 + w) of the oracle's
    own h, to one bf16 ulp (the formula, the (1 + w) gain, eps and factor placement);
  - pin_r_order: r against a numpy float32 evaluation of the reference's accumulation order (per-column sums over
    the 20 chunks, slot sums of 4, halving tree over 32 slots, rarn_final.cu:57-78), bit for bit; this is the
    only pin of the order, which no closed form fixes.
"""
from __future__ import annotations

import numpy as np

import pyoracle

D = 2560


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round-to-nearest-even (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def make_inputs(n: int, S: int, seed: int, *, pad: int = 0, scale_res: float = 1.0):
    """S partials of (n, D) stacked with a stride of n*D + pad elements, a residual and a weight, as bf16 bits."""
    rng = np.random.default_rng(seed)
    pstride = n * D + pad
    part = np.zeros(S * pstride, dtype=np.uint16)
    for s in range(S):
        part[s * pstride: s * pstride + n * D] = f32_to_bf16(rng.standard_normal(n * D).astype(np.float32) * 0.5)
    res = f32_to_bf16(rng.standard_normal((n, D)).astype(np.float32) * scale_res)
    w = f32_to_bf16(rng.standard_normal(D).astype(np.float32) * 0.1)
    return part, pstride, res, w


def h_numpy(part, S, serial, pstride, res, n):
    acc = bf16_to_f32(part[:n * D]).reshape(n, D).copy()
    for s in range(1, S):
        acc = (acc + bf16_to_f32(part[s * pstride: s * pstride + n * D]).reshape(n, D)).astype(np.float32)
        if serial:
            acc = bf16_to_f32(f32_to_bf16(acc))
    d = bf16_to_f32(f32_to_bf16(acc))
    return f32_to_bf16((bf16_to_f32(res).reshape(n, D) + d).astype(np.float32))


def r_numpy(h_bits: np.ndarray, eps: float, factor: float) -> np.ndarray:
    h = bf16_to_f32(h_bits).reshape(-1, 20, 128)
    a = np.zeros((h.shape[0], 128), dtype=np.float32)
    for k in range(20):
        a = (a + (h[:, k, :] * h[:, k, :]).astype(np.float32)).astype(np.float32)
    a4 = a.reshape(-1, 32, 4)
    sl = (((a4[:, :, 0] + a4[:, :, 1]).astype(np.float32) + a4[:, :, 2]).astype(np.float32) + a4[:, :, 3])
    sl = sl.astype(np.float32)
    half = 16
    while half >= 1:
        sl = (sl[:, :half] + sl[:, half:2 * half]).astype(np.float32)
        half //= 2
    tot = sl[:, 0]
    x = (tot * np.float32(factor)).astype(np.float32) + np.float32(eps)
    return (1.0 / np.sqrt(x.astype(np.float32).astype(np.float64))).astype(np.float32)


# --------------------------------------------------------------------------------------------------- pins

def pin_codes(mutant=0):
    part, ps, res, w = make_inputs(1, 2, 0)
    assert pyoracle.rarn(part, 2, 0, ps, res, w, 0, mutant=mutant)[0] == 0
    assert pyoracle.rarn(part, 2, 0, ps, res, w, 1, D=2048, mutant=mutant)[0] == -1
    assert pyoracle.rarn(part, 1, 0, ps, res, w, 1, mutant=mutant)[0] == -2
    assert pyoracle.rarn(part, 9, 0, ps, res, w, 1, mutant=mutant)[0] == -2


def pin_h_numpy(mutant=0):
    for S, serial, seed in [(2, 0, 1), (3, 1, 2), (5, 0, 3), (8, 1, 4)]:
        n = 5
        part, ps, res, w = make_inputs(n, S, seed, pad=24)
        code, h, _, _ = pyoracle.rarn(part, S, serial, ps, res, w, n, mutant=mutant)
        assert code == 0
        ref = h_numpy(part, S, serial, ps, res, n)
        assert np.array_equal(h.reshape(-1), ref.reshape(-1)), f"h differs (S={S}, serial={serial})"


def _one_row(vals_parts, res_val, w_val=0.0):
    S = len(vals_parts)
    part = np.concatenate([f32_to_bf16(np.full(D, v, np.float32)) for v in vals_parts])
    res = f32_to_bf16(np.full(D, res_val, np.float32))
    w = f32_to_bf16(np.full(D, w_val, np.float32))
    return part, S, D, res, w


def pin_h_rounding(mutant=0):
    e = 2.0 ** -8
    # non-serial: 1 + 2^-8 + 2^-8 = 1 + 2^-7 exactly, which bf16 holds; serial: bf16(1 + 2^-8) is a tie -> 1.0
    for serial, want in [(0, 1.0 + 2 * e), (1, 1.0)]:
        part, S, ps, res, w = _one_row([1.0, e, e], 0.0)
        h = bf16_to_f32(pyoracle.rarn(part, S, serial, ps, res, w, 1, mutant=mutant)[1])
        assert np.all(h == np.float32(want)), f"serial={serial}: h {h[0, 0]} != {want}"
    # d = bf16(1 + 2^-8) = 1.0 before the residual 2^-8 is added: h = bf16(1 + 2^-8) = 1.0 (not 1 + 2^-7)
    part, S, ps, res, w = _one_row([1.0, e], e)
    h = bf16_to_f32(pyoracle.rarn(part, S, 0, ps, res, w, 1, mutant=mutant)[1])
    assert np.all(h == 1.0), f"d must be rounded to bf16 before the residual: h {h[0, 0]}"


def pin_rms_formula(mutant=0):
    eps, factor = 1e-6, 1.0 / D
    for S, seed in [(2, 11), (4, 12)]:
        n = 6
        part, ps, res, w = make_inputs(n, S, seed)
        code, hb, ob, _ = pyoracle.rarn(part, S, 0, ps, res, w, n, eps=eps, factor=factor, mutant=mutant)
        assert code == 0
        h = bf16_to_f32(hb).astype(np.float64)
        wf = bf16_to_f32(w).astype(np.float64)
        r = 1.0 / np.sqrt(np.float64(np.float32(factor)) * (h * h).sum(axis=1, keepdims=True) + eps)
        want = h * r * (1.0 + wf)
        got = bf16_to_f32(ob).astype(np.float64)
        tol = np.abs(want) * 2.0 ** -8 + 1e-30  # one bf16 ulp (relative 2^-8 covers rounding of both)
        bad = np.abs(got - want) > tol
        assert not bad.any(), f"out off the RMSNorm formula at {int(bad.sum())} elements"
    # closed form: a constant row h = 2 (residual 2, zero partials): sum(h^2) = 4 D, r = 1/2 (factor = 1/D,
    # eps = 0), out = bf16(2 * r * (1 + w)) = 1 + w for w = 0.5 -> 1.5
    part, S, ps, res, w = _one_row([0.0, 0.0], 2.0, 0.5)
    ob = pyoracle.rarn(part, S, 0, ps, res, w, 1, eps=0.0, factor=1.0 / D, mutant=mutant)[2]
    assert np.all(bf16_to_f32(ob) == 1.5), f"constant row: out {bf16_to_f32(ob)[0, 0]} != 1.5"


def pin_r_order(mutant=0):
    eps, factor = 1e-6, 1.0 / D
    n = 64
    part, ps, res, w = make_inputs(n, 3, 21, scale_res=3.0)
    code, hb, _, r = pyoracle.rarn(part, 3, 0, ps, res, w, n, eps=eps, factor=factor, mutant=mutant)
    assert code == 0
    want = r_numpy(hb, eps, factor)
    diff = int((r.view(np.uint32) != want.view(np.uint32)).sum())
    assert diff == 0, f"r differs from the reference's accumulation order in {diff} of {n} rows"


ALL_PINS = [pin_codes, pin_h_numpy, pin_h_rounding, pin_rms_formula, pin_r_order]
