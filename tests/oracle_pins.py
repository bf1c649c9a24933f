"""Checks that pin the CPU oracle to facts it does not compute itself.

The reference ships no golden vectors or tests for this path, so each pin compares the oracle with something
independent of its code: torch's scaled_dot_product_attention / logsumexp in float64 (library routines), closed
forms (Q = 0 gives the mean of the visible V rows and LSE = log of their count; a single visible key gives V[0]
and LSE = its logit; no visible key gives 0 and -inf), structural identities (GQA fold = MHA with repeated K/V,
varlen = independent sequences, split partials + LSE combine = whole), and an exact-arithmetic sigmoid.
Every pin raises AssertionError on a mismatch; test_oracle_mutants.py shows that each deliberate oracle mistake
fails at least one of them.
"""
from __future__ import annotations

import decimal

import numpy as np

import fmha_cases as FC
import pyoracle
from reax_fmha import workloads as W

TIGHT = 1e-9


def _close(a, b, tol=TIGHT, what=""):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    ia, ib = np.isneginf(a), np.isneginf(b)
    assert (ia == ib).all(), f"{what}: -inf pattern differs"
    fin = ~ia
    if fin.any():
        d = np.nanmax(np.abs(a[fin] - b[fin]))
        assert d <= tol, f"{what}: max diff {d:.3g} > {tol}"


SDPA_CASES = [
    FC.Case("mha_causal", B=2, S=37, N=37, Hq=2, Hkv=2, D=128, mode="causal", seed=11),
    FC.Case("gqa_causal_g4", B=1, S=50, N=50, Hq=8, Hkv=2, D=128, mode="causal", seed=12),
    FC.Case("gqa_prefix_g2", B=1, S=20, N=75, Hq=4, Hkv=2, D=128, mode="causal", seed=13),  # S < N: offset causal
    FC.Case("gqa_full_d256", B=1, S=9, N=130, Hq=4, Hkv=1, D=256, mode="full", seed=14),
    FC.Case("bias_g1", B=1, S=33, N=70, Hq=2, Hkv=2, D=128, mode="bias", seed=15, bias_neg_inf_frac=0.3,
            bias_full_rows=(3,)),
]


def _qpos_case():
    rng = np.random.default_rng(16)
    S, N = 24, 40
    qp = rng.integers(-3, N + 5, size=(1, S)).astype(np.int32)
    qp[0, 0] = 0
    qp[0, 1] = -1
    qp[0, 2] = N + 10
    return FC.Case("qpos_mixed", B=1, S=S, N=N, Hq=6, Hkv=2, D=128, mode="qpos", seed=16, qpos=qp)


def pin_sdpa():
    for c in SDPA_CASES + [_qpos_case()]:
        a = FC.build(c)
        o, lse = FC.oracle_ref(c, a)
        so, slse = FC.sdpa_ref(c, a)
        _close(o, so, 1e-9, f"{c.name} O vs SDPA")
        _close(lse, slse, 1e-9, f"{c.name} LSE vs logsumexp")


def pin_closed_forms():
    c = FC.Case("closed", B=1, S=30, N=30, Hq=4, Hkv=2, D=128, mode="qpos", seed=21,
                qpos=np.array([[0, -1, 5, 29, 40, 0, 3, 7, 12, 2] * 3], dtype=np.int32))
    a = FC.build(c)
    vf = W.bf16_bits_to_f32(a["v"]).astype(np.float64)  # [B][N][Hkv][D]
    qf = W.bf16_bits_to_f32(a["q"]).astype(np.float64)
    kf = W.bf16_bits_to_f32(a["k"]).astype(np.float64)
    # (1) Q = 0: uniform weights over the visible keys
    a0 = dict(a, q=np.zeros_like(a["q"]))
    o, lse = FC.oracle_ref(c, a0)
    for m in range(c.S):
        qp = int(a["qpos"][0, m])
        for hq in range(c.Hq):
            h = hq // c.G
            if qp < 0:
                assert (o[0, m, hq] == 0).all() and np.isneginf(lse[0, hq, m]), "no visible key must give 0 / -inf"
                continue
            n = min(qp, c.N - 1) + 1
            _close(o[0, m, hq], vf[0, :n, h].mean(axis=0), 1e-12, "Q=0 mean of visible V")
            _close(lse[0, hq, m], np.log(n), 1e-12, "Q=0 LSE = log(count)")
    # (2) one visible key: O = V[0] exactly, LSE = scale * q.k0
    o, lse = FC.oracle_ref(c, a)
    for m in np.nonzero(a["qpos"][0] == 0)[0]:
        for hq in range(c.Hq):
            h = hq // c.G
            assert (o[0, m, hq] == vf[0, 0, h]).all(), "qpos = 0 must reproduce V[0] exactly"
            _close(lse[0, hq, m], c.scale * float(qf[0, m, hq] @ kf[0, 0, h]), 1e-9, "single-key LSE")
    # (3) constant V rows: O = the constant
    const = np.full_like(a["v"], 0x3FC0)  # bf16 1.5
    o, _ = FC.oracle_ref(c, dict(a, v=const))
    vis = a["qpos"][0] >= 0
    assert np.allclose(o[0, vis], 1.5, atol=1e-12, rtol=0), "constant V must give the constant"


def pin_gqa_fold():
    c = FC.Case("fold", B=1, S=40, N=40, Hq=8, Hkv=2, D=128, mode="causal", seed=31)
    a = FC.build(c)
    o, lse = FC.oracle_ref(c, a)
    cm = FC.Case("mha", B=1, S=40, N=40, Hq=8, Hkv=8, D=128, mode="causal", seed=31)
    am = dict(a, k=np.repeat(a["k"], c.G, axis=2), v=np.repeat(a["v"], c.G, axis=2))
    om, lsem = FC.oracle_ref(cm, am)
    _close(o, om, 1e-12, "GQA = MHA with repeated K/V")
    _close(lse, lsem, 1e-12, "GQA LSE")


def pin_varlen():
    c = FC.Case("varlen", B=1, S=0, N=0, Hq=4, Hkv=2, D=128, mode="varlen", seed=41, seqlens=[5, 33, 1, 64, 17])
    a = FC.build(c)
    o, lse = FC.oracle_ref(c, a)
    for b, L in enumerate(c.seqlens):
        t0 = int(a["cu"][b])
        cs = FC.Case("one", B=1, S=L, N=L, Hq=c.Hq, Hkv=c.Hkv, D=c.D, mode="causal")
        asg = dict(q=a["q"][t0:t0 + L][None], k=a["k"][t0:t0 + L][None], v=a["v"][t0:t0 + L][None],
                   qpos=np.arange(L, dtype=np.int32)[None])
        os_, ls_ = FC.oracle_ref(cs, asg)
        _close(o[t0:t0 + L], os_[0], 1e-12, f"varlen sequence {b}")
        _close(lse[t0:t0 + L], ls_[0].T, 1e-12, f"varlen LSE {b}")


def pin_split_combine():
    c = FC.Case("split", B=1, S=6, N=300, Hq=8, Hkv=2, D=128, mode="qpos", seed=51,
                qpos=np.array([[299, 150, 0, 64, 63, -1]], dtype=np.int32))
    a = FC.build(c)
    o, lse = FC.oracle_ref(c, a)
    bounds = [0, 64, 100, 192, 256, 300]
    parts = [FC.oracle_ref(c, a, key_lo=lo, key_hi=hi) for lo, hi in zip(bounds[:-1], bounds[1:])]
    po = np.stack([p[0].reshape(-1, c.D) for p in parts])  # [S][R][D], rows in (b, m, hq) order
    pl = np.stack([p[1].transpose(0, 2, 1).reshape(-1) for p in parts])  # [S][R] in (b, m, hq) order
    po = np.nan_to_num(po, nan=0.0)
    co, cl = pyoracle.lse_combine(po, pl)
    _close(co, o.reshape(-1, c.D), 1e-12, "split + combine = whole")
    _close(cl, lse.transpose(0, 2, 1).reshape(-1), 1e-12, "split LSE combine")


def exact_sigmoid_bf16(x: float) -> int:
    """Correctly rounded bf16 of 1/(1+e^-x), by 60-digit decimal arithmetic and an exact nearest-even choice
    between the two bf16 neighbours."""
    import math
    import struct

    if math.isnan(x):
        return 0x7FC0
    ctx = decimal.Context(prec=60)
    d = decimal.Decimal(x)
    if d > 400:
        s = decimal.Decimal(1)
    elif d < -400:
        s = ctx.exp(d)  # 1 + e^x == 1 to far beyond bf16 precision here
    else:
        s = ctx.divide(1, ctx.add(1, ctx.exp(-d)))
    # bf16 neighbours around s: enumerate candidates from the fp32 truncation
    f = float(s)
    u = struct.unpack("<I", struct.pack("<f", f))[0] if f != 0 else 0
    lo = u >> 16
    cands = [max(lo - 1, 0), lo, lo + 1, lo + 2]

    def val(bits):
        return decimal.Decimal(struct.unpack("<f", struct.pack("<I", bits << 16))[0])

    best = None
    for cb in cands:
        if cb >= 0x7F80:
            continue
        dist = abs(val(cb) - s)
        if best is None or dist < best[0] or (dist == best[0] and (cb & 1) == 0):
            best = (dist, cb)
    return best[1]


def pin_sigmoid(step: int = 1):
    got = pyoracle.sigmoid_bf16_all()
    xs = np.arange(0, 65536, step, dtype=np.uint32)
    xf = W.bf16_bits_to_f32(xs.astype(np.uint16))
    bad = []
    for i, x in zip(xs, xf):
        if np.isnan(x):
            assert got[i] == 0x7FC0
            continue
        e = exact_sigmoid_bf16(float(x))
        if got[i] != e:
            bad.append((int(i), int(got[i]), e))
    assert not bad, f"{len(bad)} sigmoid mismatches, first {bad[:3]}"


def pin_post():
    """V = 1 makes O = 1 exactly, so the POST output must equal the bf16 sigmoid of the gate half of qg; rows are
    scattered through inv, and inv < 0 rows leave the output untouched."""
    c = FC.Case("post", B=1, S=12, N=12, Hq=4, Hkv=2, D=128, mode="causal", seed=61)
    a = FC.build(c)
    ones = np.full_like(a["v"], 0x3F80)
    o, _ = FC.oracle_ref(c, dict(a, v=ones))
    assert (o == 1.0).all()
    G, D, Hq = c.G, c.D, c.Hq
    rng = np.random.default_rng(62)
    T = c.S + 3
    inv = rng.permutation(T)[: c.S].astype(np.int32)
    inv[4] = -1
    qg = np.zeros((T, Hq, 2 * D), dtype=np.uint16)
    qg[:, :, :D] = 0x4000  # query half: bf16 2.0 (must be ignored)
    qg[:, :, D:] = W.bf16_normal(rng, (T, Hq, D))
    out = np.full((T, Hq * D), 0x7E00, dtype=np.uint16)  # sentinel
    odense = o.transpose(0, 2, 1, 3).reshape(c.B, Hq, c.S, D)  # -> [B][Hq][S][D] then fold
    odense = odense.reshape(c.B, c.Hkv, G, c.S, D).transpose(0, 1, 3, 2, 4).reshape(c.B, c.Hkv, c.S * G, D)
    pyoracle.post_gate(odense, B=1, H=c.Hkv, G=G, M=c.S * G, D=D, inv=inv, Lq=c.S, qg=qg, qg_rs=Hq * 2 * D,
                       out=out, out_rs=Hq * D)
    sig = pyoracle.sigmoid_bf16_all()
    for m in range(c.S):
        R = inv[m]
        if R < 0:
            continue
        want = sig[qg[R, :, D:]].reshape(-1)
        assert (out[R] == want).all(), f"POST row {m}: gate half / scatter mismatch"
    written = set(int(x) for x in inv if x >= 0)
    for R in range(T):
        if R not in written:
            assert (out[R] == 0x7E00).all(), "rows not named by inv must stay untouched"


def _block_case(name, S, N, Hq, Hkv, qp, seed):
    return FC.Case(name, B=1, S=S, N=N, Hq=Hq, Hkv=Hkv, D=128, mode="qpos", seed=seed,
                   qpos=np.asarray(qp, dtype=np.int32).reshape(1, S))


def pin_block_rule():
    """The drop-in entry points' block-wide qpos = 0 rule (reax_fmha_v8.cu:155-162, 224-235), against expectations
    written out by hand: folded rows r = token*G + g of a KV head form blocks [64j, 64j + 64); a block whose largest
    raw qpos is 0 stores V[0] in every row (qpos < 0 rows included, LSE = the logit of key 0), any other block
    follows the per-row rule (qpos < 0 -> 0 / -inf)."""
    def run(c, dropin):
        a = FC.build(c)
        o, lse = FC.oracle_ref(c, a, dropin=dropin)
        qf = W.bf16_bits_to_f32(a["q"]).astype(np.float64)
        kf = W.bf16_bits_to_f32(a["k"]).astype(np.float64)
        vf = W.bf16_bits_to_f32(a["v"]).astype(np.float64)
        return a, o, lse, qf, kf, vf

    def is_v0(o, lse, qf, kf, vf, c, m, hq, what):
        h = hq // c.G
        assert (o[0, m, hq] == vf[0, 0, h]).all(), f"{what}: token {m} head {hq} must store V[0]"
        _close(lse[0, hq, m], c.scale * float(qf[0, m, hq] @ kf[0, 0, h]), 1e-9, f"{what}: LSE of key 0")

    def is_dead(o, lse, m, hq, what):
        assert (o[0, m, hq] == 0).all() and np.isneginf(lse[0, hq, m]), f"{what}: token {m} head {hq} must be 0"

    # (1) G = 8: 8 tokens per block. Block 0 = tokens 0..7 with qpos {0, -1 x 7}: every row is V[0] under the
    # drop-in rule, only token 0 under the per-row rule. Block 1 = tokens 8..15, all -1: nothing visible.
    qp = [0] + [-1] * 7 + [-1] * 8
    c = _block_case("block_g8", 16, 20, 8, 1, qp, 91)
    for dropin in (True, False):
        a, o, lse, qf, kf, vf = run(c, dropin)
        for m in range(16):
            for hq in range(8):
                if m == 0 or (dropin and m < 8):
                    is_v0(o, lse, qf, kf, vf, c, m, hq, f"g8 dropin={dropin}")
                else:
                    is_dead(o, lse, m, hq, f"g8 dropin={dropin}")
    # (2) a block whose largest qpos is 3: the per-row rule, also for the drop-in entry points
    qp = [0, -1, 3, -1, -1, -1, -1, -1]
    c = _block_case("block_max3", 8, 20, 8, 1, qp, 92)
    a, o, lse, qf, kf, vf = run(c, True)
    for hq in range(8):
        is_v0(o, lse, qf, kf, vf, c, 0, hq, "max3")
        for m in (1, 3, 4, 5, 6, 7):
            is_dead(o, lse, m, hq, "max3")
        assert np.abs(o[0, 2, hq]).sum() > 0 and np.isfinite(lse[0, hq, 2])
    # (3) G = 3: 64 is not a multiple of G, so token 21's rows 63 (g 0), 64 and 65 (g 1, 2) sit in two blocks.
    # Block 0 (rows 0..63) has largest qpos 0 (token 5), block 1 (rows 64..89) has 2 (token 25): token 21 g 0 is
    # V[0], token 21 g 1 and 2 are 0.
    qp = [-1] * 30
    qp[5], qp[25] = 0, 2
    c = _block_case("block_g3", 30, 20, 3, 1, qp, 93)
    a, o, lse, qf, kf, vf = run(c, True)
    for m in range(30):
        for g in range(3):
            r = 3 * m + g
            if r < 64:
                is_v0(o, lse, qf, kf, vf, c, m, g, "g3 block 0")
            elif m == 25:
                assert np.isfinite(lse[0, g, m])
            else:
                is_dead(o, lse, m, g, "g3 block 1")
    # (4) N = 1 and a row with qpos 5: the block's raw largest qpos is 5, not 0 (although every visible key
    # index is clamped to 0), so rows with qpos < 0 stay dead
    qp = [5, -1, -1, -1, -1, -1, -1, -1]
    c = _block_case("block_n1", 8, 1, 8, 1, qp, 94)
    a, o, lse, qf, kf, vf = run(c, True)
    for hq in range(8):
        is_v0(o, lse, qf, kf, vf, c, 0, hq, "n1")
        for m in range(1, 8):
            is_dead(o, lse, m, hq, "n1")


ALL_PINS = [pin_sdpa, pin_closed_forms, pin_gqa_fold, pin_varlen, pin_split_combine, pin_post, pin_sigmoid,
            pin_block_rule]
