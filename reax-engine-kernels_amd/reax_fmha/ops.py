"""torch-facing wrappers over the C ABI (device tensors in, device tensors out, current HIP stream).

Every call goes through libreax_howu.so / libreax_fmha_post.so; a nonzero return code raises. The tensors must
live on the GPU: there is no CPU path.
"""
from __future__ import annotations

import torch

from . import abi


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check(name: str, rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"{name} returned {rc}")


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("reax_fmha ops take device tensors only")


# ---------------------------------------------------------------------------------------------- drop-in ABI

def fmha_q(q, k, v, qpos, G, o, scale, *, lib="howu"):
    """reax_fmha_q on folded tensors: q/o [B][H][M][256] (row r = token r/G, query head h*G + r%G),
    k/v [B][N][H][256], qpos int32 [B][M/G]. Row strides are taken from the tensors."""
    _dev(q, k, v, qpos, o)
    B, H, M, D = q.shape
    N = k.shape[1]
    L = abi.howu() if lib == "howu" else abi.post()
    rc = L.reax_fmha_q(q.data_ptr(), k.data_ptr(), v.data_ptr(), qpos.data_ptr(), G, qpos.stride(0), o.data_ptr(),
                       scale, B, H, M, N, q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(2),
                       k.stride(1), v.stride(0), v.stride(2), v.stride(1), o.stride(0), o.stride(1), o.stride(2),
                       _stream())
    _check("reax_fmha_q", rc)
    return o


def fmha_b(q, k, v, bias, o, scale, *, lib="howu"):
    """reax_fmha_b: q/o [B][H][M][256], k/v [B][N][H][256], bias bf16 [B][H][M][N] (key stride 1)."""
    _dev(q, k, v, bias, o)
    B, H, M, D = q.shape
    N = k.shape[1]
    L = abi.howu() if lib == "howu" else abi.post()
    rc = L.reax_fmha_b(q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(bias), o.data_ptr(), scale, B, H, M, N,
                       q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(2), k.stride(1), v.stride(0),
                       v.stride(2), v.stride(1),
                       bias.stride(0) if bias is not None else 0, bias.stride(1) if bias is not None else 0,
                       bias.stride(2) if bias is not None else 0,
                       o.stride(0), o.stride(1), o.stride(2), _stream())
    _check("reax_fmha_b", rc)
    return o


def fmha_qp(q, k, v, qpos, G, scale, inv, Lq, qg, out):
    """reax_fmha_qp (libreax_fmha_post.so): q [B][H][M][256] folded, k/v [B][N][H][256], inv int32 [B][Lq],
    qg bf16 [T][Hq][512] (gate = second half), out bf16 [T][Hq*256]."""
    _dev(q, k, v, qpos, inv, qg, out)
    B, H, M, D = q.shape
    N = k.shape[1]
    rc = abi.post().reax_fmha_qp(q.data_ptr(), k.data_ptr(), v.data_ptr(), qpos.data_ptr(), G, qpos.stride(0),
                                 scale, B, H, M, N, q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(2),
                                 k.stride(1), v.stride(0), v.stride(2), v.stride(1), inv.data_ptr(), Lq,
                                 qg.data_ptr(), qg.stride(0), out.data_ptr(), out.stride(0), _stream())
    _check("reax_fmha_qp", rc)
    return out


# ---------------------------------------------------------------------------------------------- extensions

def attention(q, k, v, qpos, *, scale, o=None, lse=None, want_lse=True):
    """reax_fmha_qx on natural layouts: q [B][S][Hq][D], k/v [B][N][Hkv][D], qpos int32 [B][S]
    (token m sees keys 0..qpos[b][m]). Returns (o [B][S][Hq][D] bf16, lse [B][Hq][S] fp32 or None)."""
    _dev(q, k, v, qpos)
    B, S, Hq, D = q.shape
    N, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    if o is None:
        o = torch.empty_like(q)
    if want_lse and lse is None:
        lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    ls = lse.stride() if lse is not None else (0, 0, 0)
    rc = abi.howu().reax_fmha_qx(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), qpos.data_ptr(), G, qpos.stride(0), o.data_ptr(), _ptr(lse),
        scale, B, Hkv, S * G, N, D,
        q.stride(0), G * q.stride(2), q.stride(1), q.stride(2),
        k.stride(0), k.stride(2), k.stride(1), v.stride(0), v.stride(2), v.stride(1),
        o.stride(0), G * o.stride(2), o.stride(1), o.stride(2),
        ls[0], G * ls[1], ls[2], ls[1], _stream())
    _check("reax_fmha_qx", rc)
    return o, lse


def attention_varlen(q, k, v, cu_seqlens, max_seqlen, *, scale, o=None, lse=None, want_lse=True):
    """reax_fmha_varlen: q/o [T][Hq][D], k/v [T][Hkv][D], cu_seqlens int32 [nseq+1] on the device.
    Returns (o, lse [T][Hq] fp32 or None)."""
    _dev(q, k, v, cu_seqlens)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    nseq = cu_seqlens.numel() - 1
    if o is None:
        o = torch.empty_like(q)
    if want_lse and lse is None:
        lse = torch.empty((T, Hq), dtype=torch.float32, device=q.device)
    ls = lse.stride() if lse is not None else (0, 0)
    rc = abi.howu().reax_fmha_varlen(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), cu_seqlens.data_ptr(), nseq, max_seqlen, o.data_ptr(), _ptr(lse),
        scale, Hq, Hkv, D, q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        o.stride(0), o.stride(1), ls[0], ls[1], _stream())
    _check("reax_fmha_varlen", rc)
    return o, lse


def splitkv_workspace_bytes(B, Hkv, M, D, num_splits) -> int:
    return abi.howu().reax_fmha_splitkv_workspace(B, Hkv, M, D, num_splits)


def attention_splitkv(q, k, v, qpos, *, scale, num_splits, ws=None, o=None, lse=None, want_lse=True):
    """reax_fmha_splitkv on natural layouts (as attention()); ws is a uint8 device tensor (allocated if None)."""
    _dev(q, k, v, qpos)
    B, S, Hq, D = q.shape
    N, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    M = S * G
    need = splitkv_workspace_bytes(B, Hkv, M, D, num_splits)
    if ws is None:
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    if o is None:
        o = torch.empty_like(q)
    if want_lse and lse is None:
        lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    ls = lse.stride() if lse is not None else (0, 0, 0)
    rc = abi.howu().reax_fmha_splitkv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), qpos.data_ptr(), G, qpos.stride(0), o.data_ptr(), _ptr(lse),
        scale, B, Hkv, M, N, D, num_splits, ws.data_ptr(), ws.numel(),
        q.stride(0), G * q.stride(2), q.stride(1), q.stride(2),
        k.stride(0), k.stride(2), k.stride(1), v.stride(0), v.stride(2), v.stride(1),
        o.stride(0), G * o.stride(2), o.stride(1), o.stride(2),
        ls[0], G * ls[1], ls[2], ls[1], _stream())
    _check("reax_fmha_splitkv", rc)
    return o, lse


def attention_splitkv_noalloc(q, k, v, qpos, *, scale, num_splits, o, lse=None):
    """reax_fmha_splitkv_noalloc on natural layouts (as attention_splitkv): the library's static per-GPU scratch
    is the workspace, so the call allocates nothing; o (and lse, if wanted) must be given."""
    _dev(q, k, v, qpos, o, lse)
    B, S, Hq, D = q.shape
    N, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    ls = lse.stride() if lse is not None else (0, 0, 0)
    rc = abi.howu().reax_fmha_splitkv_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), qpos.data_ptr(), G, qpos.stride(0), o.data_ptr(), _ptr(lse),
        scale, B, Hkv, S * G, N, D, num_splits,
        q.stride(0), G * q.stride(2), q.stride(1), q.stride(2),
        k.stride(0), k.stride(2), k.stride(1), v.stride(0), v.stride(2), v.stride(1),
        o.stride(0), G * o.stride(2), o.stride(1), o.stride(2),
        ls[0], G * ls[1], ls[2], ls[1], _stream())
    _check("reax_fmha_splitkv_noalloc", rc)
    return o, lse


def rarn(part, S, serial, pstride, res, w, n, *, eps, factor, h_out=None, out=None, D=2560):
    """reax_rarn (libreax_howu/reax_rarn_final.cu:98-106) on device tensors: part is a bf16 buffer holding S
    partials of (n, D) rows, pstride elements apart; res (n, D), w (D,). Returns (h_out, out), each (n, D) bf16."""
    _dev(part, res, w)
    if h_out is None:
        h_out = torch.empty((max(n, 1), D), dtype=torch.bfloat16, device=res.device)
    if out is None:
        out = torch.empty((max(n, 1), D), dtype=torch.bfloat16, device=res.device)
    rc = abi.howu().reax_rarn(part.data_ptr(), S, int(serial), pstride, res.data_ptr(), w.data_ptr(),
                              h_out.data_ptr(), out.data_ptr(), n, D, eps, factor, _stream())
    _check("reax_rarn", rc)
    return h_out, out


def conv_l2(qkv, cache, meta, w, *, Tf, KD, VD, eps, rep=1, skip_v=0, RT=16, q=None, k=None, v=None):
    """reax_conv_l2 (libreax_howu/reax_conv_v2.cu:164-181) on device tensors: qkv (rows, SX) and cache (rows, C)
    bf16, meta int32 (Tf, 4), w bf16 (2*KD + VD, 4). Returns (q, k, v): q, k (Tf, rep*KD), v (Tf, VD) bf16."""
    _dev(qkv, cache, meta, w)
    REP = 1 if rep == 1 else 2
    dev = qkv.device
    q = torch.empty((max(Tf, 1), REP * KD), dtype=torch.bfloat16, device=dev) if q is None else q
    k = torch.empty((max(Tf, 1), REP * KD), dtype=torch.bfloat16, device=dev) if k is None else k
    v = torch.empty((max(Tf, 1), max(VD, 1)), dtype=torch.bfloat16, device=dev) if v is None else v
    rc = abi.howu().reax_conv_l2(qkv.data_ptr(), qkv.stride(0), cache.data_ptr(), cache.stride(0), meta.data_ptr(),
                                 w.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), Tf, eps, KD, VD, rep, skip_v,
                                 RT, _stream())
    _check("reax_conv_l2", rc)
    return q, k, v


def conv_v(qkv, cache, meta, w, *, Tf, KD, VD, v=None):
    """reax_conv_v (libreax_howu/reax_conv_v2.cu:183-189): the value channels only. Returns v (Tf, VD) bf16."""
    _dev(qkv, cache, meta, w)
    v = torch.empty((max(Tf, 1), VD), dtype=torch.bfloat16, device=qkv.device) if v is None else v
    rc = abi.howu().reax_conv_v(qkv.data_ptr(), qkv.stride(0), cache.data_ptr(), cache.stride(0), meta.data_ptr(),
                                w.data_ptr(), v.data_ptr(), Tf, KD, VD, _stream())
    _check("reax_conv_v", rc)
    return v


def kkt(k, g, beta, cu, cidx, *, NT, H, HV, A=None):
    """reax_kkt (libreax_howu/reax_kkt.cu:263-270) on device tensors: k bf16 [T][H][128], g fp32 [T][HV], beta bf16
    [T][HV], cu / cidx int64. Writes A (bf16 [T][HV][64], allocated if None: entries outside the lower block
    triangle stay as allocated) and returns it."""
    _dev(k, g, beta, cu, cidx)
    if A is None:
        A = torch.zeros((k.shape[0], HV, 64), dtype=torch.bfloat16, device=k.device)
    rc = abi.howu().reax_kkt(k.data_ptr(), g.data_ptr(), beta.data_ptr(), A.data_ptr(), cu.data_ptr(),
                             cidx.data_ptr(), NT, H, HV, _stream())
    _check("reax_kkt", rc)
    return A


def howu(q, k, v, beta, A, g, cu, *, N, H, HV, scale, o=None, dense=False):
    """reax_howu (skip form) or howu3_dense (libreax_howu/reax_howu.cu:349-376) on device tensors: q, k bf16
    [T][H][128], v bf16 [T][HV][128], beta bf16 [T][HV], A bf16 [T][HV][64] (the chunk solve's output), g fp32
    [T][HV] (chunk-local cumulative log2 decay), cu int64 [N+1]. Returns o, bf16 [T][HV][128]."""
    _dev(q, k, v, beta, A, g, cu)
    if o is None:
        o = torch.empty((q.shape[0], HV, 128), dtype=torch.bfloat16, device=q.device)
    fn = abi.howu().howu3_dense if dense else abi.howu().reax_howu
    rc = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), A.data_ptr(), g.data_ptr(), o.data_ptr(),
            cu.data_ptr(), scale, N, H, HV, _stream())
    _check("reax_howu", rc)
    return o


def howu_norm(q, k, v, beta, A, g, cu, f2s, z, nw, *, N, H, HV, scale, eps, factor, out):
    """reax_howu_norm (libreax_howu/reax_howu_norm_v3.cu:431-435): the chunked forward with the fused gated-RMSNorm
    epilogue; token t writes row f2s[t] of out (bf16 [rows][HV][128]); z: gate bf16 [rows][HV*128] (row stride
    z.stride(0)); nw: norm weight bf16 [128]. Returns out."""
    _dev(q, k, v, beta, A, g, cu, f2s, z, nw, out)
    rc = abi.howu().reax_howu_norm(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), A.data_ptr(),
                                   g.data_ptr(), out.data_ptr(), cu.data_ptr(), scale, N, H, HV, _stream(),
                                   f2s.data_ptr(), z.data_ptr(), z.stride(0), nw.data_ptr(), eps, factor)
    _check("reax_howu_norm", rc)
    return out


# ---------------------------------------------------------------------------------------------- GEMM libraries

def _rowmajor_bf16(*ts):
    for t in ts:
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1 or t.stride(0) != t.shape[1]:
            raise ValueError("GEMM operands are contiguous row-major bf16 matrices")


def gemm(x, w, *, cfg=0, d=None):
    """reax_gemm (libreax_plain/gemm_plain2.cu:37-56): d = bf16(x w^T), x bf16 [M][K], w bf16 [N][K]; d bf16 [M][ldd]
    with ldd >= N (allocated [M][N] if None; its row stride is d.stride(0)). Returns d."""
    _dev(x, w, d)
    _rowmajor_bf16(x, w)
    M, K = x.shape
    N = w.shape[0]
    if d is None:
        d = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if d.dtype != torch.bfloat16 or d.stride(1) != 1 or d.shape[0] != M or d.shape[1] < N:
        raise ValueError("d must be bf16 [M][>= N] with unit column stride")
    _check("reax_gemm", abi.plain().reax_gemm(cfg, x.data_ptr(), w.data_ptr(), d.data_ptr(), M, N, K, d.stride(0),
                                              _stream()))
    return d


def slices(x, w, *, kps, S, part_fp32=True, cfg=0, p=None):
    """reax_slices (libreax_slices/gemm_slices_v2.cu:65-84): the split-K partials p[s] = x[:, s kps:(s+1) kps]
    w[:, s kps:(s+1) kps]^T for s < S, fp32 or bf16 [S][M][N] (allocated if None). Returns p."""
    _dev(x, w, p)
    _rowmajor_bf16(x, w)
    M, K = x.shape
    N = w.shape[0]
    dt = torch.float32 if part_fp32 else torch.bfloat16
    if p is None:
        p = torch.empty((S, M, N), dtype=dt, device=x.device)
    if p.dtype != dt or not p.is_contiguous() or tuple(p.shape) != (S, M, N):
        raise ValueError(f"p must be contiguous {dt} [S][M][N]")
    _check("reax_slices", abi.slices().reax_slices(cfg, int(part_fp32), x.data_ptr(), w.data_ptr(), p.data_ptr(), M,
                                                   N, kps, S, K, _stream()))
    return p


def gv(x, w_g4, *, cfg=0, out=None):
    """reax_gv (libreax_gv/gateup_vis2.cu:184-208): out = bf16(bf16(silu(bf16 g)) bf16 u) with g, u the gate and up
    columns of x w_g4^T, w_g4 bf16 [2 N2][K] holding gate and up rows interleaved in groups of 4. Returns out,
    bf16 [M][N2]."""
    _dev(x, w_g4, out)
    _rowmajor_bf16(x, w_g4)
    M, K = x.shape
    N2 = w_g4.shape[0] // 2
    if out is None:
        out = torch.empty((M, N2), dtype=torch.bfloat16, device=x.device)
    if out.dtype != torch.bfloat16 or not out.is_contiguous() or tuple(out.shape) != (M, N2):
        raise ValueError("out must be contiguous bf16 [M][N2]")
    _check("reax_gv", abi.gv().reax_gv(cfg, x.data_ptr(), w_g4.data_ptr(), out.data_ptr(), M, N2, K, _stream()))
    return out
