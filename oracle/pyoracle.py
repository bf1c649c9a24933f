"""ctypes binding of the CPU oracle (liboracle_fmha.so, and liboracle_gdn.so for the norm kernels).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check in __graft_entry__.py and by the cpu_baseline
leg of bench.py, always as the checker (or the timed CPU baseline), never as the product path.

All array arguments are numpy arrays; bf16 tensors travel as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_fmha.so")
GDN_LIB_PATH = os.path.join(HERE, "liboracle_gdn.so")

MASK_QPOS, MASK_BIAS, MASK_VARLEN_CAUSAL, MASK_NONE = 0, 1, 2, 3

MUTANTS = {
    "no_scale": 1,
    "gqa_head_major": 2,
    "causal_strict": 3,
    "no_normalise": 4,
    "lse_log2": 5,
    "sigmoid_sign": 6,
    "gate_query_half": 7,
    "combine_no_weight": 8,
    "block_tokens": 9,
    "block_clamped": 10,
    "block_off": 11,
}


class Args(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("qpos", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("cu_seqlens", ctypes.c_void_p),
        ("qpBs", ctypes.c_int64),
        ("bsB", ctypes.c_int64), ("bsH", ctypes.c_int64), ("bsM", ctypes.c_int64),
        ("qsB", ctypes.c_int64), ("qsH", ctypes.c_int64), ("qsT", ctypes.c_int64), ("qsG", ctypes.c_int64),
        ("ksB", ctypes.c_int64), ("ksH", ctypes.c_int64), ("ksM", ctypes.c_int64),
        ("vsB", ctypes.c_int64), ("vsH", ctypes.c_int64), ("vsM", ctypes.c_int64),
        ("mask_mode", ctypes.c_int32),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("G", ctypes.c_int32),
        ("M", ctypes.c_int32), ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("key_lo", ctypes.c_int32), ("key_hi", ctypes.c_int32), ("p_bf16", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("qpos0_block", ctypes.c_int32),
    ]


_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_attn_f64.restype = ctypes.c_int
        L.oracle_attn_f64.argtypes = [ctypes.POINTER(Args), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_int32, ctypes.c_int32]
        L.oracle_attn_f32.restype = ctypes.c_int
        L.oracle_attn_f32.argtypes = L.oracle_attn_f64.argtypes
        L.oracle_set_mutant.argtypes = [ctypes.c_int32]
        L.oracle_get_mutant.restype = ctypes.c_int32
        L.oracle_f64_to_bf16.restype = ctypes.c_uint16
        L.oracle_f64_to_bf16.argtypes = [ctypes.c_double]
        L.oracle_f64_to_bf16_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_sigmoid_bf16.restype = ctypes.c_uint16
        L.oracle_sigmoid_bf16.argtypes = [ctypes.c_uint16]
        L.oracle_sigmoid_bf16_all.argtypes = [ctypes.c_void_p]
        L.oracle_post_gate.restype = ctypes.c_int
        L.oracle_post_gate.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                       ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_lse_combine.restype = ctypes.c_int
        L.oracle_lse_combine.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
        L.oracle_args_size.restype = ctypes.c_int32
        assert L.oracle_args_size() == ctypes.sizeof(Args), "oracle Args layout mismatch"
        _lib = L
    return _lib


def set_mutant(name_or_id) -> None:
    mid = MUTANTS[name_or_id] if isinstance(name_or_id, str) else int(name_or_id)
    lib().oracle_set_mutant(mid)


def _ptr(a):
    return None if a is None else a.ctypes.data


def _u16(a):
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, a.dtype
    return a


def attention(q, k, v, *, G, B, H, M, N, D, scale, strides, mask_mode=MASK_QPOS, qpos=None, qpBs=0,
              bias=None, bias_strides=(0, 0, 0), cu_seqlens=None, key_lo=0, key_hi=0, p_bf16=False,
              rows=None, precision="f64", nthreads=None, qpos0_block=False):
    """Runs the oracle on flat uint16 (bf16 bits) buffers q, k, v addressed through `strides`:
    strides = dict(qsB, qsH, qsT, qsG, ksB, ksH, ksM, vsB, vsH, vsM), all in elements.

    Returns (o, lse) as dense arrays o[B][H][M][D], lse[B][H][M] (float64 or float32). Entries of rows not
    computed (outside `rows`, or beyond a varlen sequence) are NaN. qpos0_block selects the drop-in entry points'
    block-wide qpos = 0 rule (reax_fmha_q / reax_fmha_qp); the extension entry points use the per-row rule.
    """
    L = lib()
    q, k, v = _u16(q), _u16(k), _u16(v)
    keep = [q, k, v]
    a = Args()
    a.q, a.k, a.v = _ptr(q), _ptr(k), _ptr(v)
    if qpos is not None:
        qpos = np.ascontiguousarray(qpos, dtype=np.int32)
        keep.append(qpos)
        a.qpos = _ptr(qpos)
    if bias is not None:
        bias = _u16(bias)
        keep.append(bias)
        a.bias = _ptr(bias)
    if cu_seqlens is not None:
        cu_seqlens = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        keep.append(cu_seqlens)
        a.cu_seqlens = _ptr(cu_seqlens)
    a.qpBs = qpBs
    a.bsB, a.bsH, a.bsM = bias_strides
    for name in ("qsB", "qsH", "qsT", "qsG", "ksB", "ksH", "ksM", "vsB", "vsH", "vsM"):
        setattr(a, name, int(strides[name]))
    a.mask_mode = mask_mode
    a.B, a.H, a.G, a.M, a.N, a.D = B, H, G, M, N, D
    a.key_lo, a.key_hi = key_lo, key_hi
    a.p_bf16 = 1 if p_bf16 else 0
    a.scale = scale
    a.qpos0_block = 1 if qpos0_block else 0
    dt = np.float64 if precision == "f64" else np.float32
    o = np.full((B, H, M, D), np.nan, dtype=dt)
    lse = np.full((B, H, M), np.nan, dtype=dt)
    rr = None
    nr = 0
    if rows is not None:
        rr = np.ascontiguousarray(rows, dtype=np.int32)
        nr = len(rr)
        keep.append(rr)
    nt = nthreads if nthreads else (os.cpu_count() or 1)
    fn = L.oracle_attn_f64 if precision == "f64" else L.oracle_attn_f32
    rc = fn(ctypes.byref(a), o.ctypes.data, lse.ctypes.data, _ptr(rr), nr, nt)
    if rc != 0:
        raise ValueError(f"oracle rejected arguments (rc={rc})")
    return o, lse


def f64_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f64_to_bf16_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


def sigmoid_bf16_all() -> np.ndarray:
    out = np.empty(65536, dtype=np.uint16)
    lib().oracle_sigmoid_bf16_all(out.ctypes.data)
    return out


def post_gate(o, *, B, H, G, M, D, inv, Lq, qg, qg_rs, out, out_rs):
    """Applies the POST epilogue to a dense oracle output o[B][H][M][D] in place into `out` (uint16)."""
    o = np.ascontiguousarray(o, dtype=np.float64)
    inv = np.ascontiguousarray(inv, dtype=np.int32)
    qg = _u16(qg)
    assert out.dtype == np.uint16 and out.flags.c_contiguous
    rc = lib().oracle_post_gate(o.ctypes.data, B, H, G, M, D, inv.ctypes.data, Lq, qg.ctypes.data, qg_rs,
                                out.ctypes.data, out_rs)
    if rc != 0:
        raise ValueError("oracle_post_gate rejected arguments")
    return out


def lse_combine(part_o, part_lse):
    """part_o[S][R][D], part_lse[S][R] -> (o[R][D], lse[R])."""
    part_o = np.ascontiguousarray(part_o, dtype=np.float64)
    part_lse = np.ascontiguousarray(part_lse, dtype=np.float64)
    S, R, D = part_o.shape
    o = np.empty((R, D))
    lse = np.empty(R)
    rc = lib().oracle_lse_combine(part_o.ctypes.data, part_lse.ctypes.data, S, R, D, o.ctypes.data, lse.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_lse_combine rejected arguments")
    return o, lse


# ------------------------------------------------------------------------------------------- norm kernels

_gdn = None

RARN_MUTANTS = {"rarn_flat_sum": 1, "rarn_no_one_plus_w": 2, "rarn_no_d_round": 3}


def gdn_lib():
    global _gdn
    if _gdn is None:
        if not os.path.exists(GDN_LIB_PATH):
            build()
        L = ctypes.CDLL(GDN_LIB_PATH)
        L.oracle_rarn.restype = ctypes.c_int
        L.oracle_rarn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_longlong, ctypes.c_void_p,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
        _gdn = L
    return _gdn


def rarn(part, S, serial, pstride, res, w, n, *, D=2560, eps=1e-6, factor=1.0 / 2560, mutant=0):
    """reax_rarn on the CPU: returns (code, h_out, out, r): h_out and out as uint16 bf16 bit arrays of shape (n, D),
    r the per-row fp32 reciprocal RMS."""
    part = np.ascontiguousarray(part, dtype=np.uint16)
    res = np.ascontiguousarray(res, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    h_out = np.zeros((max(n, 0), D), dtype=np.uint16)
    out = np.zeros((max(n, 0), D), dtype=np.uint16)
    r = np.zeros(max(n, 0), dtype=np.float32)
    m = RARN_MUTANTS.get(mutant, mutant) if isinstance(mutant, str) else mutant
    code = gdn_lib().oracle_rarn(_ptr(part), S, int(serial), pstride, _ptr(res), _ptr(w), _ptr(h_out), _ptr(out),
                                 n, D, ctypes.c_float(eps), ctypes.c_float(factor), m, _ptr(r))
    return code, h_out, out, r


CONV_MUTANTS = {"conv_taps_reversed": 1, "conv_route_strict": 2, "conv_flat_l2": 3, "conv_silu_sign": 4}


def conv(qkv, SX, cache, C, meta, w, Tf, *, KD, VD, eps=1e-6, rep=1, skip_v=0, u0=0, units=None, mutant=0):
    """reax_conv_l2 / reax_conv_v on the CPU. qkv, cache, w: bf16 bit arrays; meta: int32 [Tf][4].
    Returns (q, k, v, rstd): q, k of shape (Tf, rep*KD) and v (Tf, VD) as bf16 bits (zeros where not written),
    rstd (Tf, 2*KD/128) fp32."""
    L = gdn_lib()
    if not hasattr(L, "_conv_typed"):
        L.oracle_conv.restype = ctypes.c_int
        L.oracle_conv.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                  ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        L._conv_typed = True
    qkv = np.ascontiguousarray(qkv, dtype=np.uint16)
    cache = np.ascontiguousarray(cache, dtype=np.uint16)
    meta = np.ascontiguousarray(meta, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    REP = 1 if rep == 1 else 2
    q = np.zeros((Tf, REP * KD), dtype=np.uint16)
    k = np.zeros((Tf, REP * KD), dtype=np.uint16)
    v = np.zeros((Tf, max(VD, 1)), dtype=np.uint16)
    nqk = 2 * KD // 128
    rstd = np.zeros((Tf, nqk), dtype=np.float32)
    if units is None:
        units = nqk + (0 if skip_v else VD // 128)
    m = CONV_MUTANTS.get(mutant, mutant) if isinstance(mutant, str) else mutant
    L.oracle_conv(_ptr(qkv), SX, _ptr(cache), C, _ptr(meta), _ptr(w), _ptr(q), _ptr(k), _ptr(v), Tf,
                  ctypes.c_float(eps), KD, VD, rep, skip_v, u0, units, m, _ptr(rstd))
    return q, k, v, rstd


KKT_MUTANTS = {"kkt_decay_sign": 1, "kkt_beta_column": 2, "kkt_diag_in_m": 3, "kkt_sign": 4}


def kkt(k, g, beta, cu, cidx, *, NT, H, HV, A=None, mutant=0):
    """reax_kkt on the CPU (double precision): k bf16 bits [T][H][128], g fp32 [T][HV], beta bf16 bits [T][HV],
    cu / cidx int64. Writes into A (bf16 bits [T][HV][64], allocated zero-filled if None); returns (code, A)."""
    L = gdn_lib()
    if not hasattr(L, "_kkt_typed"):
        L.oracle_kkt.restype = ctypes.c_int
        L.oracle_kkt.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 4
        L._kkt_typed = True
    k = np.ascontiguousarray(k, dtype=np.uint16)
    g = np.ascontiguousarray(g, dtype=np.float32)
    beta = np.ascontiguousarray(beta, dtype=np.uint16)
    cu = np.ascontiguousarray(cu, dtype=np.int64)
    cidx = np.ascontiguousarray(cidx, dtype=np.int64)
    if A is None:
        A = np.zeros((k.shape[0], HV, 64), dtype=np.uint16)
    m = KKT_MUTANTS.get(mutant, mutant) if isinstance(mutant, str) else mutant
    code = L.oracle_kkt(_ptr(k), _ptr(g), _ptr(beta), _ptr(A), _ptr(cu), _ptr(cidx), NT, H, HV, m)
    return code, A


HOWU_MUTANTS = {"howu_inter_no_decay": 1, "howu_strict_causal": 2, "howu_state_no_decay": 3, "howu_vdec_no_decay": 4}


def howu(q, k, v, beta, A, g, cu, *, N, H, HV, scale, exact=False, o=None, mutant=0):
    """reax_howu on the CPU: q, k bf16 bits [T][H][128], v bf16 [T][HV][128], beta bf16 [T][HV], A bf16 [T][HV][64]
    (ignored when exact), g fp32 [T][HV] (chunk-local cumulative log2 decay), cu int64. Returns o, bf16 bits
    [T][HV][128] (rows written for every token)."""
    L = gdn_lib()
    if not hasattr(L, "_howu_typed"):
        L.oracle_howu.restype = ctypes.c_int
        L.oracle_howu.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                          ctypes.c_int, ctypes.c_int]
        L._howu_typed = True
    arrs = [np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v, beta)]
    A = np.ascontiguousarray(A if A is not None else np.zeros((q.shape[0], HV, 64)), dtype=np.uint16)
    g = np.ascontiguousarray(g, dtype=np.float32)
    cu = np.ascontiguousarray(cu, dtype=np.int64)
    if o is None:
        o = np.zeros((q.shape[0], HV, 128), dtype=np.uint16)
    m = HOWU_MUTANTS.get(mutant, mutant) if isinstance(mutant, str) else mutant
    code = L.oracle_howu(_ptr(arrs[0]), _ptr(arrs[1]), _ptr(arrs[2]), _ptr(arrs[3]), _ptr(A), _ptr(g), _ptr(o),
                         _ptr(cu), ctypes.c_float(scale), N, H, HV, int(exact), m)
    assert code == 0, code
    return o
