"""Attention test cases shared by the CPU pins and the GPU parity tests.

A case is stored in natural layouts: q [B][S][Hq][D], k/v [B][N][Hkv][D] (uint16 bf16 bits), qpos [B][S] int32
(qpos mode), bias [B][Hkv][M][N] bf16 bits over folded rows (bias mode, G = 1 as reax_fmha_b uses), or packed
[T][H][D] with cu_seqlens (varlen). Reference results come back as o [B][S][Hq][D] float64, lse [B][Hq][S].
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import pyoracle
from reax_fmha import workloads as W

NEG_INF = -np.inf


@dataclass
class Case:
    name: str
    B: int
    S: int
    N: int
    Hq: int
    Hkv: int
    D: int
    mode: str = "causal"  # causal | qpos | bias | varlen | full
    seed: int = 0
    qpos: np.ndarray | None = None
    seqlens: list = field(default_factory=list)
    bias_neg_inf_frac: float = 0.0
    bias_full_rows: tuple = ()  # folded rows whose bias is -inf everywhere

    @property
    def G(self):
        return self.Hq // self.Hkv

    @property
    def scale(self):
        # the C ABI passes the scale as fp32 (v8:444); every reference result uses that same rounded value
        return float(np.float32(1.0 / np.sqrt(self.D)))


def build(c: Case) -> dict:
    rng = np.random.default_rng(c.seed)
    if c.mode == "varlen":
        T = sum(c.seqlens)
        q = W.bf16_normal(rng, (T, c.Hq, c.D))
        k = W.bf16_normal(rng, (T, c.Hkv, c.D))
        v = W.bf16_normal(rng, (T, c.Hkv, c.D))
        cu = np.zeros(len(c.seqlens) + 1, dtype=np.int32)
        cu[1:] = np.cumsum(c.seqlens)
        return dict(q=q, k=k, v=v, cu=cu)
    q = W.bf16_normal(rng, (c.B, c.S, c.Hq, c.D))
    k = W.bf16_normal(rng, (c.B, c.N, c.Hkv, c.D))
    v = W.bf16_normal(rng, (c.B, c.N, c.Hkv, c.D))
    out = dict(q=q, k=k, v=v)
    if c.mode == "causal":
        out["qpos"] = np.tile(np.arange(c.S, dtype=np.int32) + (c.N - c.S), (c.B, 1))
    elif c.mode == "full":
        out["qpos"] = np.full((c.B, c.S), c.N - 1, dtype=np.int32)
    elif c.mode == "qpos":
        out["qpos"] = np.ascontiguousarray(c.qpos, dtype=np.int32).reshape(c.B, c.S)
    elif c.mode == "bias":
        assert c.G == 1, "bias mode follows reax_fmha_b: G = 1"
        b = rng.standard_normal((c.B, c.Hkv, c.S, c.N)).astype(np.float32)
        if c.bias_neg_inf_frac > 0:
            b[rng.random(b.shape) < c.bias_neg_inf_frac] = -np.inf
        for r in c.bias_full_rows:
            b[:, :, r, :] = -np.inf
        u = b.view(np.uint32)
        out["bias"] = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return out


def oracle_ref(c: Case, a: dict, *, rows=None, precision="f64", p_bf16=False, key_lo=0, key_hi=0, dropin=False):
    """(o [B][S][Hq][D], lse [B][Hq][S]) from the CPU oracle; for varlen o [T][Hq][D], lse [T][Hq]. dropin: the
    drop-in entry points' block-wide qpos = 0 rule (reax_fmha_q / reax_fmha_qp)."""
    if c.mode == "varlen":
        T = sum(c.seqlens)
        L = max(c.seqlens)
        st = dict(qsB=0, qsH=c.G * c.D, qsT=c.Hq * c.D, qsG=c.D, ksB=0, ksH=c.D, ksM=c.Hkv * c.D,
                  vsB=0, vsH=c.D, vsM=c.Hkv * c.D)
        o, lse = pyoracle.attention(a["q"], a["k"], a["v"], G=c.G, B=len(c.seqlens), H=c.Hkv, M=L * c.G, N=L,
                                    D=c.D, scale=c.scale, strides=st, mask_mode=pyoracle.MASK_VARLEN_CAUSAL,
                                    cu_seqlens=a["cu"], rows=rows, precision=precision, p_bf16=p_bf16)
        on = np.full((T, c.Hq, c.D), np.nan)
        ln = np.full((T, c.Hq), np.nan)
        for b, Lb in enumerate(c.seqlens):
            t0 = a["cu"][b]
            ob = o[b, :, : Lb * c.G].reshape(c.Hkv, Lb, c.G, c.D).transpose(1, 0, 2, 3).reshape(Lb, c.Hq, c.D)
            lb = lse[b, :, : Lb * c.G].reshape(c.Hkv, Lb, c.G).transpose(1, 0, 2).reshape(Lb, c.Hq)
            on[t0:t0 + Lb] = ob
            ln[t0:t0 + Lb] = lb
        return on, ln
    st = W.natural_strides(c.B, c.S, c.Hq, c.N, c.Hkv, c.D)
    kw = {}
    if c.mode == "bias":
        kw = dict(mask_mode=pyoracle.MASK_BIAS, bias=a["bias"],
                  bias_strides=(c.Hkv * c.S * c.N, c.S * c.N, c.N))
    else:
        kw = dict(mask_mode=pyoracle.MASK_QPOS, qpos=a["qpos"], qpBs=c.S, qpos0_block=dropin)
    o, lse = pyoracle.attention(a["q"], a["k"], a["v"], G=c.G, B=c.B, H=c.Hkv, M=c.S * c.G, N=c.N, D=c.D,
                                scale=c.scale, strides=st, rows=rows, precision=precision, p_bf16=p_bf16,
                                key_lo=key_lo, key_hi=key_hi, **kw)
    return W.folded_to_natural(o, c.S, c.G), W.folded_lse_to_natural(lse, c.S, c.G)


def visible_mask(c: Case, a: dict) -> np.ndarray:
    """bool [B][Hq][S][N]: key j visible to (b, query head, token m) under the case's mask."""
    if c.mode == "bias":
        raise ValueError("bias mode has no boolean mask")
    qp = a["qpos"].astype(np.int64)  # [B][S]
    j = np.arange(c.N)
    vis = (j[None, None, :] <= qp[:, :, None])  # [B][S][N]
    return np.broadcast_to(vis[:, None, :, :], (c.B, c.Hq, c.S, c.N))


def sdpa_ref(c: Case, a: dict):
    """(o, lse) from torch's scaled_dot_product_attention in float64 on the CPU (a library routine independent
    of the oracle); LSE from torch.logsumexp of the masked, scaled logits. Rows that see nothing get O = 0,
    LSE = -inf (the reference semantics, v8:303, 331-334), where SDPA itself would return NaN."""
    import torch

    f = lambda x: torch.from_numpy(W.bf16_bits_to_f32(x).astype(np.float64))
    q = f(a["q"]).permute(0, 2, 1, 3)  # [B][Hq][S][D]
    k = f(a["k"]).permute(0, 2, 1, 3).repeat_interleave(c.G, dim=1)
    v = f(a["v"]).permute(0, 2, 1, 3).repeat_interleave(c.G, dim=1)
    if c.mode == "bias":
        bias = torch.from_numpy(W.bf16_bits_to_f32(a["bias"]).astype(np.float64))  # [B][H][S][N] (G = 1)
        add = bias
    else:
        vis = torch.from_numpy(np.ascontiguousarray(visible_mask(c, a)))
        add = torch.zeros(vis.shape, dtype=torch.float64).masked_fill(~vis, float("-inf"))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=add, scale=c.scale)
    logits = torch.matmul(q, k.transpose(-1, -2)) * c.scale + add
    lse = torch.logsumexp(logits, dim=-1)
    dead = torch.isinf(lse) & (lse < 0)
    o = torch.where(dead[..., None], torch.zeros_like(o), o)
    return o.permute(0, 2, 1, 3).numpy(), lse.numpy()


def check_tolerance(o_gpu_bits: np.ndarray, o_ref: np.ndarray, lse_gpu=None, lse_ref=None, *,
                    max_abs=2e-2, mean_abs=2e-3, lse_rel=1e-3, where=""):
    """The parity bar: bf16 outputs within max-abs 2e-2 and mean-abs 2e-3 of the double oracle; LSE within
    1e-3 relative: |dLSE| <= 1e-3 * |LSE| + 1e-5 (the 1e-5 absolute term only matters where LSE is within 1e-2 of 0,
    where a relative bound alone would ask for more than fp32 resolution); -inf LSE must match exactly. Returns a
    dict of the measured errors (lse_rel = max |dLSE| / (|LSE| + 1e-2))."""
    og = W.bf16_bits_to_f32(o_gpu_bits).astype(np.float64)
    sel = ~np.isnan(o_ref)
    assert np.isfinite(og[sel]).all(), f"{where}: non-finite GPU output"
    err = np.abs(og[sel] - o_ref[sel])
    res = dict(max_abs=float(err.max()) if err.size else 0.0, mean_abs=float(err.mean()) if err.size else 0.0)
    assert res["max_abs"] <= max_abs, f"{where}: max-abs {res['max_abs']:.3g} > {max_abs}"
    assert res["mean_abs"] <= mean_abs, f"{where}: mean-abs {res['mean_abs']:.3g} > {mean_abs}"
    if lse_gpu is not None:
        lsel = ~np.isnan(lse_ref)
        lr, lg = lse_ref[lsel], np.asarray(lse_gpu, dtype=np.float64)[lsel]
        ninf = np.isneginf(lr)
        assert (np.isneginf(lg) == ninf).all(), f"{where}: -inf LSE rows differ"
        d = np.abs(lg[~ninf] - lr[~ninf])
        lim = lse_rel * np.abs(lr[~ninf]) + 1e-5
        res["lse_rel"] = float((d / (np.abs(lr[~ninf]) + 1e-2)).max()) if d.size else 0.0
        if d.size:
            worst = int(np.argmax(d - lim))
            assert (d <= lim).all(), (f"{where}: LSE off by {d[worst]:.3g} at LSE {lr[~ninf][worst]:.6g} "
                                      f"(bound 1e-3 relative)")
    return res
