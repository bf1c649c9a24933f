"""Inputs and independent checks for the causal conv + SiLU + L2 norm (reax_conv_l2 / reax_conv_v,
libreax_howu/reax_conv_v2.cu).

The pins fix what the oracle must compute without re-running its code path:
  - pin_onehot: with every channel's weight 1 on tap J and 0 elsewhere, a v output is bf16(silu(x)) of the source
    row that tap J reads (position meta.x - 3 + J, from qkv at or above meta.y, from the cache below it, zero before
    position 0), against float64 SiLU to one bf16 ulp (tap order, routing and its boundary, SiLU, conv_v2:88-122);
  - pin_general: random weights: v outputs against float64 SiLU of the bf16-rounded exact tap sum, to two bf16 ulps;
  - pin_l2: q/k outputs against s / sqrt(eps + sum(s^2)) in float64 to two bf16 ulps, and rep 2 writes each head
    twice (conv_v2:123-142);
  - pin_l2_order: rstd against a numpy float32 evaluation of the reference's order (s1*s1, then fma of s0, s2..s7
    per 8-channel group, butterfly over group distance 8, 4, 2, 1), bit for bit: the only pin of that order.
"""
from __future__ import annotations

import numpy as np

import pyoracle
from rarn_cases import bf16_to_f32, f32_to_bf16


def make_inputs(seqs, KD, VD, seed, *, pad=8, onehot=None):
    """seqs: list of (cached positions L, new tokens n). Returns a dict with qkv (rows = new tokens), cache (3 rows
    per sequence: its last min(L, 3) positions), meta [Tf][4], w [channels][4] and the strides."""
    rng = np.random.default_rng(seed)
    ch = 2 * KD + VD
    SX = C = ch + pad
    Tf = sum(n for _, n in seqs)
    qkv = f32_to_bf16(rng.standard_normal((Tf, SX)).astype(np.float32))
    # 3 rows per sequence, plus 3 spare rows so that a planted routing mistake in the oracle stays in bounds
    cache = f32_to_bf16(rng.standard_normal((3 * len(seqs) + 3, C)).astype(np.float32))
    meta = np.zeros((Tf, 4), dtype=np.int32)
    row = 0
    for i, (L, n) in enumerate(seqs):
        lo = max(L - 3, 0)
        for j in range(n):
            # position L + j; positions >= L are this call's rows (qkv row = row_of_first_new + pos - L),
            # positions < L come from the cache rows 3i .. 3i + 2 holding positions lo .. L - 1
            meta[row + j] = (L + j, L, row - L, 3 * i - lo)
        row += n
    if onehot is None:
        w = f32_to_bf16((rng.standard_normal((ch, 4)) * 0.5).astype(np.float32))
    else:
        wf = np.zeros((ch, 4), dtype=np.float32)
        wf[:, onehot] = 1.0
        w = f32_to_bf16(wf)
    return dict(qkv=qkv, SX=SX, cache=cache, C=C, meta=meta, w=w, Tf=Tf, KD=KD, VD=VD, seqs=seqs)


def source_values(a, J):
    """Float64 value read by tap J for every token and channel (0 where the position is negative)."""
    Tf, ch = a["Tf"], 2 * a["KD"] + a["VD"]
    x = np.zeros((Tf, ch))
    qf, cf = bf16_to_f32(a["qkv"]).astype(np.float64), bf16_to_f32(a["cache"]).astype(np.float64)
    for t in range(Tf):
        mx, my, mz, mw = a["meta"][t]
        src = mx - 3 + J
        if src < 0:
            continue
        x[t] = qf[mz + src, :ch] if src >= my else cf[mw + src, :ch]
    return x


def silu64(y):
    return y / (1.0 + np.exp(-y))


def run(a, *, rep=1, skip_v=0, eps=1e-6, mutant=0, **kw):
    return pyoracle.conv(a["qkv"], a["SX"], a["cache"], a["C"], a["meta"], a["w"], a["Tf"], KD=a["KD"], VD=a["VD"],
                         eps=eps, rep=rep, skip_v=skip_v, mutant=mutant, **kw)


def _ulps_ok(got_bits, want, nulp):
    got = bf16_to_f32(got_bits).astype(np.float64)
    tol = np.abs(want) * (nulp * 2.0 ** -8) + 1e-30
    return np.abs(got - want) <= tol


SEQS = [(0, 5), (1, 2), (2, 3), (7, 4), (3, 1)]


def pin_onehot(mutant=0):
    for J in range(4):
        a = make_inputs(SEQS, 128, 256, 30 + J, onehot=J)
        _, _, v, _ = run(a, mutant=mutant)
        x = source_values(a, J)[:, 2 * a["KD"]:]
        want = silu64(x)
        ok = _ulps_ok(v, want, 1)
        assert ok.all(), f"tap {J}: {int((~ok).sum())} v outputs off bf16(silu(source))"


def pin_general(mutant=0):
    a = make_inputs(SEQS, 128, 256, 41)
    _, _, v, _ = run(a, mutant=mutant)
    wf = bf16_to_f32(a["w"]).astype(np.float64)
    acc = sum(source_values(a, J) * wf[None, :, J] for J in range(4))
    y = bf16_to_f32(f32_to_bf16(acc.astype(np.float32))).astype(np.float64)
    want = silu64(y)[:, 2 * a["KD"]:]
    ok = _ulps_ok(v, want, 2)
    assert ok.all(), f"{int((~ok).sum())} v outputs off silu(bf16(conv))"


def pin_l2(mutant=0):
    eps = 1e-6
    for rep in (1, 2):
        a = make_inputs(SEQS, 256, 128, 52 + rep)
        KD = a["KD"]
        q, k, _, _ = run(a, rep=rep, eps=eps, mutant=mutant)
        wf = bf16_to_f32(a["w"]).astype(np.float64)
        acc = sum(source_values(a, J) * wf[None, :, J] for J in range(4))
        y = bf16_to_f32(f32_to_bf16(acc.astype(np.float32))).astype(np.float64)
        s = bf16_to_f32(f32_to_bf16(silu64(y).astype(np.float32))).astype(np.float64)
        for name, out, off in (("q", q, 0), ("k", k, KD)):
            for h in range(KD // 128):
                sh = s[:, off + 128 * h: off + 128 * (h + 1)]
                want = sh / np.sqrt(eps + (sh * sh).sum(axis=1, keepdims=True))
                for copy in range(rep):
                    col = (rep * h + copy) * 128
                    ok = _ulps_ok(out[:, col: col + 128], want, 2)
                    assert ok.all(), f"rep {rep} {name} head {h} copy {copy}: {int((~ok).sum())} outputs off"


def pin_l2_order(mutant=0):
    eps = 1e-6
    a = make_inputs(SEQS, 256, 0, 61)
    _, _, _, rstd = run(a, eps=eps, mutant=mutant)
    wf = bf16_to_f32(a["w"]).astype(np.float32)
    # s recomputed in numpy float32 (fma chain as one rounding of an exact float64 sum, bf16 rounding, SiLU with
    # 1 + exp(-y) rounded to fp32), then the reference's sum order
    Tf, ch = a["Tf"], 2 * a["KD"]
    acc = np.zeros((Tf, ch), dtype=np.float32)
    for J in range(4):
        x = source_values(a, J).astype(np.float32)
        acc = (acc.astype(np.float64) + (wf[None, :ch, J].astype(np.float64) * x)).astype(np.float32)
    y = bf16_to_f32(f32_to_bf16(acc))
    d = (1.0 + np.exp(-y.astype(np.float64))).astype(np.float32)
    s = bf16_to_f32(f32_to_bf16((y / d).astype(np.float32)))
    g = s.reshape(Tf, ch // 128, 16, 8)
    p = (g[..., 1] * g[..., 1]).astype(np.float32)
    for i in [0] + list(range(2, 8)):
        p = (p.astype(np.float64) + g[..., i].astype(np.float64) ** 2).astype(np.float32)  # exact square, one rounding
    for dist in (8, 4, 2, 1):
        p = (p + p[..., np.arange(16) ^ dist]).astype(np.float32)
    want = (1.0 / np.sqrt((np.float32(eps) + p[..., 0]).astype(np.float32).astype(np.float64))).astype(np.float32)
    diff = int((rstd.view(np.uint32) != want.view(np.uint32)).sum())
    assert diff == 0, f"rstd differs from the reference's order at {diff} of {rstd.size} (token, head) pairs"


ALL_PINS = [pin_onehot, pin_general, pin_l2, pin_l2_order]
