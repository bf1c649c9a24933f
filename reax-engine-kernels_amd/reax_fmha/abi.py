"""ctypes bindings of libreax_howu.so and libreax_fmha_post.so.

This is the binding the REAX engine's Python loader makes for the reference libraries (dlopen by path, argtypes
exactly as the C prototypes: c_void_p for pointers and the stream, c_int, c_longlong, c_float). The prototypes
are the reference's (libreax_howu/reax_fmha_v8.cu:434-450, libreax_fmha_post/reax_fmha_v11.cu:565-590) plus the
extension entry points declared in include/libreax_howu.h.

Loading fails loudly when a library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# always the in-tree build: no environment variable redirects the product loader to another build
LIB_DIR = os.path.join(PKG_ROOT, "lib")
HOWU_PATH = os.path.join(LIB_DIR, "libreax_howu.so")
POST_PATH = os.path.join(LIB_DIR, "libreax_fmha_post.so")

P, I, LL, F, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float, ctypes.c_size_t

# name -> argtypes (restype c_int unless listed in RESTYPES)
SIGNATURES = {
    "reax_fmha_b": [P, P, P, P, P, F, I, I, I, I] + [LL] * 15 + [P],
    "reax_fmha_q": [P, P, P, P, I, LL, P, F, I, I, I, I] + [LL] * 12 + [P],
    "reax_fmha_qp": [P, P, P, P, I, LL, F, I, I, I, I] + [LL] * 9 + [P, I, P, LL, P, LL, P],
    "reax_fmha_qx": [P, P, P, P, I, LL, P, P, F, I, I, I, I, I] + [LL] * 18 + [P],
    "reax_fmha_varlen": [P, P, P, P, I, I, P, P, F, I, I, I] + [LL] * 10 + [P],
    "reax_fmha_splitkv_workspace": [I, I, I, I, I],
    "reax_fmha_splitkv": [P, P, P, P, I, LL, P, P, F, I, I, I, I, I, I, P, SZ] + [LL] * 18 + [P],
    "reax_fmha_splitkv_noalloc": [P, P, P, P, I, LL, P, P, F, I, I, I, I, I, I] + [LL] * 18 + [P],
    "howu3_dense": [P, P, P, P, P, P, P, P, F, I, I, I, P],
    "howu3_skip": [P, P, P, P, P, P, P, P, F, I, I, I, P],
    "howu3_smem": [],
    "reax_howu": [P, P, P, P, P, P, P, P, F, I, I, I, P],
    "reax_kkt": [P, P, P, P, P, P, I, I, I, P],
    "reax_kkt_smem": [],
    "reax_rarn": [P, I, I, LL, P, P, P, P, I, I, F, F, P],
    "reax_howu_norm": [P, P, P, P, P, P, P, P, F, I, I, I, P, P, P, LL, P, F, F],
    "reax_conv_l2": [P, LL, P, I, P, P, P, P, P, I, F, I, I, I, I, I, P],
    "reax_conv_v": [P, LL, P, I, P, P, P, I, I, I, P],
    # the GEMM libraries (libreax_plain.so, libreax_slices.so, libreax_gv.so)
    "reax_gemm_ncfg": [],
    "reax_gemm_cfgname": [I],
    "reax_gemm": [I, P, P, P, I, I, I, I, P],
    "reax_slices_ncfg": [],
    "reax_slices_cfgname": [I],
    "reax_slices": [I, I, P, P, P, I, I, I, I, I, P],
    "reax_gv_ncfg": [],
    "reax_gv_cfgname": [I],
    "reax_gv": [I, P, P, P, I, I, I, P],
}
RESTYPES = {"reax_fmha_splitkv_workspace": SZ, "reax_gemm_cfgname": ctypes.c_char_p,
            "reax_slices_cfgname": ctypes.c_char_p, "reax_gv_cfgname": ctypes.c_char_p}

HOWU_SYMBOLS = ["reax_fmha_b", "reax_fmha_q", "reax_fmha_qx", "reax_fmha_varlen", "reax_fmha_splitkv_workspace",
                "reax_fmha_splitkv", "reax_fmha_splitkv_noalloc", "howu3_dense", "howu3_skip", "howu3_smem", "reax_howu", "reax_kkt",
                "reax_kkt_smem", "reax_rarn", "reax_howu_norm", "reax_conv_l2", "reax_conv_v"]
POST_SYMBOLS = ["reax_fmha_b", "reax_fmha_q", "reax_fmha_qp"]
PLAIN_SYMBOLS = ["reax_gemm_ncfg", "reax_gemm_cfgname", "reax_gemm"]
SLICES_SYMBOLS = ["reax_slices_ncfg", "reax_slices_cfgname", "reax_slices"]
GV_SYMBOLS = ["reax_gv_ncfg", "reax_gv_cfgname", "reax_gv"]
PLAIN_PATH = os.path.join(LIB_DIR, "libreax_plain.so")
SLICES_PATH = os.path.join(LIB_DIR, "libreax_slices.so")
GV_PATH = os.path.join(LIB_DIR, "libreax_gv.so")


_cache: dict[str, ctypes.CDLL] = {}


def _load(path: str, symbols: list[str]) -> ctypes.CDLL:
    if path in _cache:
        return _cache[path]
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() (make -C reax-engine-kernels_amd)")
    lib = ctypes.CDLL(path)
    for name in symbols:
        fn = getattr(lib, name)
        fn.argtypes = SIGNATURES[name]
        fn.restype = RESTYPES.get(name, I)
    _cache[path] = lib
    return lib


def howu() -> ctypes.CDLL:
    """libreax_howu.so with every exported entry point typed."""
    return _load(HOWU_PATH, HOWU_SYMBOLS)


def post() -> ctypes.CDLL:
    """libreax_fmha_post.so with its three entry points typed."""
    return _load(POST_PATH, POST_SYMBOLS)


def plain() -> ctypes.CDLL:
    """libreax_plain.so (reax_gemm)."""
    return _load(PLAIN_PATH, PLAIN_SYMBOLS)


def slices() -> ctypes.CDLL:
    """libreax_slices.so (reax_slices)."""
    return _load(SLICES_PATH, SLICES_SYMBOLS)


def gv() -> ctypes.CDLL:
    """libreax_gv.so (reax_gv)."""
    return _load(GV_PATH, GV_SYMBOLS)
