"""The benchmark configurations of the FMHA path and seeded synthetic inputs for them.

Inputs are i.i.d. N(0,1) draws from numpy's PCG64 generator with a recorded seed, rounded to bf16 (RNE), so the
same arrays can be rebuilt on any host for the CPU oracle. Work counting: FLOPs = 4*Hq*D*P where P is the number
of (query, key) pairs the mask admits (causal: sum_seq S(S+1)/2); decode bytes = K + V + Q + O + LSE.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E


@dataclass
class Config:
    name: str
    kind: str  # "prefill" | "varlen" | "decode" | "post"
    B: int
    S: int     # query tokens per sequence (prefill), 1 for decode
    N: int     # keys per sequence
    Hq: int
    Hkv: int
    D: int
    seed: int
    num_splits: int = 0
    nseq: int = 0
    seqlens: list = field(default_factory=list)

    @property
    def G(self) -> int:
        return self.Hq // self.Hkv

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.D)

    def pairs(self) -> int:
        if self.kind == "varlen":
            return sum(L * (L + 1) // 2 for L in self.seqlens)
        if self.kind == "decode":
            return self.B * self.S * self.N
        return self.B * self.S * (self.S + 1) // 2

    def flops(self) -> int:
        return 4 * self.Hq * self.D * self.pairs()

    def decode_bytes(self) -> int:
        kv = 2 * self.B * self.N * self.Hkv * self.D * 2
        if self.kind == "decode_post":
            # the drop-in reax_fmha_qp: Q read, the gate half of qg read, the gated output written; no LSE
            return kv + 3 * self.B * self.S * self.Hq * self.D * 2
        qo = 2 * self.B * self.S * self.Hq * self.D * 2
        return kv + qo + self.B * self.S * self.Hq * 4


def varlen_lengths(seed: int, nseq: int = 8, lo: int = 256, hi: int = 2048) -> list:
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=nseq)]


CONFIGS = {
    1: Config("c1_causal_gqa_s512_d128", "prefill", B=1, S=512, N=512, Hq=8, Hkv=2, D=128, seed=1001),
    2: Config("c2_causal_gqa_s4096_d128", "prefill", B=1, S=4096, N=4096, Hq=32, Hkv=8, D=128, seed=1002),
    3: Config("c3_varlen_causal_gqa_d128", "varlen", B=1, S=0, N=0, Hq=16, Hkv=4, D=128, seed=1003, nseq=8,
              seqlens=varlen_lengths(1003)),
    4: Config("c4_decode_splitkv_kv8192_d128", "decode", B=16, S=1, N=8192, Hq=32, Hkv=8, D=128, seed=1004,
              num_splits=16),
    5: Config("c5_causal_gqa_s32768_d256_gated", "post", B=1, S=32768, N=32768, Hq=16, Hkv=2, D=256, seed=1005),
}

# The engine's per-token decode call through the drop-in reax_fmha_qp (config 5's model: Hq 16, Hkv 2, D 256, the
# sigmoid gate): one query token per sequence (Lq 1 x G 8 = 8 folded rows per KV head) over a 32768-key cache, at
# batch 1 and 16. Memory-bound: reported in HBM GB/s of K + V + Q + gate + output.
DROPIN_DECODE = {
    B: Config(f"qp_decode_b{B}_kv32768_d256_gated", "decode_post", B=B, S=1, N=32768, Hq=16, Hkv=2, D=256,
              seed=1006 + B)
    for B in (1, 16)
}


def bf16_normal(rng: np.random.Generator, shape) -> np.ndarray:
    """N(0,1) float32 draws rounded to bf16 (RNE); returned as uint16 bit patterns."""
    x = rng.standard_normal(size=shape, dtype=np.float32)
    u = x.view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bits_to_torch(a: np.ndarray, device=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return t.to(device) if device is not None else t


def torch_to_bits(t) -> np.ndarray:
    import torch

    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bf16_bits_to_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def make_prefill_inputs(cfg: Config):
    """q [B][S][Hq][D], k/v [B][N][Hkv][D] as uint16 bf16 bits, qpos [B][S] = causal (token m sees 0..m)."""
    rng = np.random.default_rng(cfg.seed)
    q = bf16_normal(rng, (cfg.B, cfg.S, cfg.Hq, cfg.D))
    k = bf16_normal(rng, (cfg.B, cfg.N, cfg.Hkv, cfg.D))
    v = bf16_normal(rng, (cfg.B, cfg.N, cfg.Hkv, cfg.D))
    off = cfg.N - cfg.S
    qpos = np.tile(np.arange(cfg.S, dtype=np.int32) + off, (cfg.B, 1))
    return q, k, v, qpos


def make_gate(cfg: Config):
    """Gate logits [S][Hq][D] N(0,1) bf16 (after q, k, v in the same stream of draws)."""
    rng = np.random.default_rng(cfg.seed + 7)
    return bf16_normal(rng, (cfg.B * cfg.S, cfg.Hq, cfg.D))


def make_varlen_inputs(cfg: Config):
    rng = np.random.default_rng(cfg.seed)
    T = sum(cfg.seqlens)
    q = bf16_normal(rng, (T, cfg.Hq, cfg.D))
    k = bf16_normal(rng, (T, cfg.Hkv, cfg.D))
    v = bf16_normal(rng, (T, cfg.Hkv, cfg.D))
    cu = np.zeros(len(cfg.seqlens) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(cfg.seqlens)
    return q, k, v, cu


def make_decode_inputs(cfg: Config):
    """q [B][1][Hq][D]; contiguous KV cache k/v [B][N][Hkv][D]; qpos [B][1] = N-1 (every cached key visible)."""
    rng = np.random.default_rng(cfg.seed)
    q = bf16_normal(rng, (cfg.B, cfg.S, cfg.Hq, cfg.D))
    k = bf16_normal(rng, (cfg.B, cfg.N, cfg.Hkv, cfg.D))
    v = bf16_normal(rng, (cfg.B, cfg.N, cfg.Hkv, cfg.D))
    qpos = np.full((cfg.B, cfg.S), cfg.N - 1, dtype=np.int32)
    return q, k, v, qpos


def natural_strides(B, S, Hq, N, Hkv, D):
    """Oracle strides (elements) for q [B][S][Hq][D], k/v [B][N][Hkv][D] with the folded row r = m*G + g."""
    G = Hq // Hkv
    return dict(qsB=S * Hq * D, qsH=G * D, qsT=Hq * D, qsG=D,
                ksB=N * Hkv * D, ksH=D, ksM=Hkv * D, vsB=N * Hkv * D, vsH=D, vsM=Hkv * D)


def folded_to_natural(o_dense: np.ndarray, S: int, G: int) -> np.ndarray:
    """Dense oracle output [B][Hkv][S*G][D] -> [B][S][Hq][D]."""
    B, Hkv, M, D = o_dense.shape
    return o_dense.reshape(B, Hkv, S, G, D).transpose(0, 2, 1, 3, 4).reshape(B, S, Hkv * G, D)


def folded_lse_to_natural(lse_dense: np.ndarray, S: int, G: int) -> np.ndarray:
    """Dense oracle LSE [B][Hkv][S*G] -> [B][Hq][S]."""
    B, Hkv, M = lse_dense.shape
    return lse_dense.reshape(B, Hkv, S, G).transpose(0, 1, 3, 2).reshape(B, Hkv * G, S)
