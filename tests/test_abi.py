"""CPU: the drop-in boundary. The two libraries load, export exactly the functions their headers declare (the
reference's names plus the declared extensions), set no soname, bind every argument with the ctypes type of its C
prototype, and return the documented codes for calls that touch no GPU (NULL bias, the argument guards of the GDN /
norm / conv entry points, workspace sizing)."""
import ctypes
import os
import re
import subprocess

import pytest

from reax_fmha import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")


def declared(header):
    text = open(os.path.join(INC, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(\w+)\s*\(", text, flags=re.M)))


def exported_functions(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    return sorted(line.split()[-1] for line in out.splitlines() if line.split()[1] == "T")


@pytest.mark.parametrize("path,header,names", [
    (abi.HOWU_PATH, "libreax_howu.h", abi.HOWU_SYMBOLS),
    (abi.POST_PATH, "libreax_fmha_post.h", abi.POST_SYMBOLS),
])
def test_exports_match_header(path, header, names):
    assert os.path.exists(path), f"{path} not built"
    decl = declared(header)
    assert decl == sorted(names), "header and binding disagree"
    assert exported_functions(path) == decl


def test_reference_names_present():
    # reference: libreax_howu.so exports reax_fmha_b/q (v8:435, 444) and the GDN symbols; fmha_post its three
    assert {"reax_fmha_b", "reax_fmha_q", "howu3_dense", "howu3_skip", "howu3_smem", "reax_howu", "reax_kkt",
            "reax_kkt_smem", "reax_rarn", "reax_howu_norm", "reax_conv_l2", "reax_conv_v"} <= set(abi.HOWU_SYMBOLS)
    assert abi.POST_SYMBOLS == ["reax_fmha_b", "reax_fmha_q", "reax_fmha_qp"]


@pytest.mark.parametrize("path", [abi.HOWU_PATH, abi.POST_PATH, abi.PLAIN_PATH, abi.SLICES_PATH, abi.GV_PATH])
def test_hip_imports_resolve_in_torch_runtime(path):
    # The libraries are loaded into processes whose HIP runtime may be an older one (torch's bundled
    # libamdhip64.so, loaded first): every versioned HIP symbol they import must be defined there, or dlopen fails
    torch = pytest.importorskip("torch")
    rt = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
    if not os.path.exists(rt):
        pytest.skip("torch has no bundled HIP runtime")
    nm = lambda *a: subprocess.run(["nm", "-D", *a], check=True, capture_output=True, text=True).stdout
    have = {line.split()[-1].replace("@@", "@") for line in nm("--defined-only", rt).splitlines()}
    need = [line.split()[-1] for line in nm("--undefined-only", path).splitlines() if "@hip_" in line]
    assert need, "no HIP imports found"
    missing = [sym for sym in need if sym not in have]
    assert not missing, f"{os.path.basename(path)} imports HIP symbols torch's runtime lacks: {missing}"


@pytest.mark.parametrize("path", [abi.HOWU_PATH, abi.POST_PATH])
def test_no_soname(path):
    out = subprocess.run(["readelf", "-d", path], check=True, capture_output=True, text=True).stdout
    assert "SONAME" not in out


@pytest.mark.parametrize("loader", [abi.howu, abi.post])
def test_null_bias_returns_minus_one(loader):
    L = loader()
    args = [None] * 3 + [None, None, ctypes.c_float(0.1), 1, 1, 1, 1] + [0] * 15 + [None]
    assert L.reax_fmha_b(*args) == -1  # v8:439: returns before any launch


@pytest.mark.parametrize("loader", [abi.howu, abi.post])
def test_fmha_empty_grid(loader):
    # an empty query block or batch: hipErrorInvalidConfiguration (9), the code of the reference's own launch with a
    # zero-sized grid; returned before any HIP call (the buffers are never touched, so aligned stand-in addresses do)
    L = loader()
    q, k, v, qpos, o = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    strides = [8 * 256, 256, 256] * 4  # qs/ks/vs/os B, H, M: multiples of 8 elements
    q_args = lambda B, M: [q, k, v, qpos, 1, 0, o, ctypes.c_float(0.0625), B, 1, M, 16] + strides + [None]
    assert L.reax_fmha_q(*q_args(1, 0)) == 9
    assert L.reax_fmha_q(*q_args(0, 64)) == 9
    assert L.reax_fmha_q(*q_args(0, 200)) == 9  # more than 64 rows: the wavefront-pair kernel's launcher
    if loader is abi.howu:
        x_args = lambda B, M, D: [q, k, v, qpos, 1, 0, o, None, ctypes.c_float(0.0625), B, 1, M, 16, D] + [8 * D] * 18 + [None]
        assert L.reax_fmha_qx(*x_args(1, 0, 128)) == 9
        assert L.reax_fmha_qx(*x_args(1, 0, 256)) == 9
        assert L.reax_fmha_qx(*x_args(0, 300, 128)) == 9  # the persistent head_dim-128 kernel's launcher
        assert L.reax_fmha_qx(*x_args(0, 300, 256)) == 9


def test_rarn_argument_codes():
    # reax_rarn (rarn_final.cu:100, 104): n <= 0 -> 0 (even with a wrong D), D != 2560 -> -1, S outside 2..8 -> -2;
    # a missing buffer (which the reference would fault on) -> hipErrorInvalidValue; none of these launches
    L = abi.howu()
    args = lambda S, n, D: (None, S, 0, 0, None, None, None, None, n, D, 1e-6, 1.0 / 2560, None)
    assert L.reax_rarn(*args(2, 0, 2560)) == 0
    assert L.reax_rarn(*args(2, -3, 100)) == 0
    assert L.reax_rarn(*args(2, 4, 2048)) == -1
    assert L.reax_rarn(*args(1, 4, 2560)) == -2
    assert L.reax_rarn(*args(9, 4, 2560)) == -2
    assert L.reax_rarn(*args(4, 4, 2560)) == 1  # hipErrorInvalidValue


def test_conv_argument_codes():
    # reax_conv_l2 / reax_conv_v (conv_v2:166, 173-177, 185): Tf <= 0 -> 0, RT outside {8, 16, 32} -> -1; missing
    # buffers (which the reference would fault on) -> hipErrorInvalidValue; none of these launches
    L = abi.howu()
    l2 = lambda Tf, RT: (None, 0, None, 0, None, None, None, None, None, Tf, 1e-6, 128, 128, 1, 0, RT, None)
    assert L.reax_conv_l2(*l2(0, 16)) == 0
    assert L.reax_conv_l2(*l2(0, 7)) == 0
    assert L.reax_conv_l2(*l2(4, 12)) == -1
    assert L.reax_conv_l2(*l2(4, 16)) == 1
    assert L.reax_conv_v(None, 0, None, 0, None, None, None, 0, 128, 128, None) == 0
    assert L.reax_conv_v(None, 0, None, 0, None, None, None, 3, 128, 128, None) == 1


def test_kkt_argument_codes():
    # reax_kkt: HV != 2H -> -1 (kkt:265); an empty grid -> hipErrorInvalidConfiguration (the reference's launch
    # error); missing buffers -> hipErrorInvalidValue; none of these launches. reax_kkt_smem: the kernel's LDS bytes
    L = abi.howu()
    assert L.reax_kkt(*([None] * 6 + [1, 2, 3, None])) == -1
    assert L.reax_kkt(*([None] * 6 + [0, 2, 4, None])) == 9
    assert L.reax_kkt(*([None] * 6 + [3, 2, 4, None])) == 1
    assert 0 < L.reax_kkt_smem() <= 160 * 1024


def test_howu_argument_codes():
    # reax_howu / howu3_skip / howu3_dense: an empty grid -> hipErrorInvalidConfiguration (the reference's launch
    # error); H not dividing HV or missing buffers -> hipErrorInvalidValue; howu3_smem: the kernel's LDS bytes
    L = abi.howu()
    for fn in (L.reax_howu, L.howu3_skip, L.howu3_dense):
        assert fn(*([None] * 8 + [1.0, 0, 1, 2, None])) == 9
        assert fn(*([None] * 8 + [1.0, 1, 3, 2, None])) == 1
        assert fn(*([None] * 8 + [1.0, 1, 1, 2, None])) == 1
    assert 0 < L.howu3_smem() <= 160 * 1024
    norm = lambda N, H, HV: [None] * 6 + [None, None, 1.0, N, H, HV, None, None, None, 0, None, 1e-6, 1.0]
    assert L.reax_howu_norm(*norm(0, 1, 2)) == 9
    assert L.reax_howu_norm(*norm(1, 3, 2)) == 1
    assert L.reax_howu_norm(*norm(1, 1, 2)) == 1


@pytest.mark.parametrize("loader,symbols,path", [("plain", "PLAIN_SYMBOLS", "PLAIN_PATH"),
                                                  ("slices", "SLICES_SYMBOLS", "SLICES_PATH"),
                                                  ("gv", "GV_SYMBOLS", "GV_PATH")])
def test_gemm_libraries_export_and_no_soname(loader, symbols, path):
    # reference: libreax_plain.so / libreax_slices.so / libreax_gv.so export exactly their ncfg / cfgname / run
    # symbols (gemm_plain2.cu:31-37, gemm_slices_v2.cu:55-65, gateup_vis2.cu:172-182), no soname
    getattr(abi, loader)()
    out = subprocess.run(["nm", "-D", "--defined-only", getattr(abi, path)], check=True, capture_output=True,
                         text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert exported == set(getattr(abi, symbols))
    dyn = subprocess.run(["readelf", "-d", getattr(abi, path)], check=True, capture_output=True, text=True).stdout
    assert "SONAME" not in dyn


def test_gemm_argument_codes():
    # config counts and names; an unknown cfg -> 9; shapes the reference's kernels cannot take -> 1 (plain, slices:
    # CUTLASS can_implement; gv: K % 8 or N2 % 4, gv:143) or 3 (gv: an empty grid fails to launch); none launches
    P, S, G = abi.plain(), abi.slices(), abi.gv()
    assert (P.reax_gemm_ncfg(), S.reax_slices_ncfg(), G.reax_gv_ncfg()) == (15, 16, 20)
    assert P.reax_gemm_cfgname(15) == b"?" and S.reax_slices_cfgname(-1) == b"?" and G.reax_gv_cfgname(20) == b"?"
    assert P.reax_gemm_cfgname(0) != b"?" and S.reax_slices_cfgname(15) != b"?" and G.reax_gv_cfgname(19) != b"?"
    assert P.reax_gemm(15, None, None, None, 8, 8, 8, 8, None) == 9
    assert P.reax_gemm(0, None, None, None, 8, 8, 8, 8, None) == 1          # missing buffers
    assert S.reax_slices(16, 1, None, None, None, 8, 8, 8, 1, 8, None) == 9
    assert S.reax_slices(0, 1, None, None, None, 8, 8, 8, 2, 8, None) == 1  # S * kps > K
    assert G.reax_gv(20, None, None, None, 8, 8, 8, None) == 9
    assert G.reax_gv(0, None, None, None, 8, 8, 12, None) == 1              # K % 8
    assert G.reax_gv(0, None, None, None, 8, 6, 8, None) == 1               # N2 % 4
    assert G.reax_gv(0, None, None, None, 0, 8, 8, None) == 3               # empty grid
    assert G.reax_gv(0, None, None, None, 8, 2 ** 30 + 4, 8, None) == 3     # 2 N2 beyond int


def test_splitkv_noalloc_rejects_oversize():
    # partials of B 64 x 8 KV heads x 64 splits x 4 rows x 129 floats (67.6 MB) exceed the 8 MiB static scratch:
    # hipErrorOutOfMemory before any HIP call; a NULL qpos is hipErrorInvalidValue as for reax_fmha_splitkv
    L = abi.howu()
    dummy = ctypes.c_int(0)
    args = [None, None, None, ctypes.addressof(dummy), 4, 1, None, None, 0.088, 64, 8, 4, 8192, 128, 64] + [0] * 18
    assert L.reax_fmha_splitkv_noalloc(*args, None) == 2
    args[3] = None
    assert L.reax_fmha_splitkv_noalloc(*args, None) == 1


def test_splitkv_workspace_size():
    L = abi.howu()
    # config 4: B 16, Hkv 8, M = G = 4 rows, D 128, 16 splits: partial O fp32 + LSE fp32, each 256-byte aligned
    rows = 16 * 8 * 16 * 4
    want = -(-rows * 128 * 4 // 256) * 256 + -(-rows * 4 // 256) * 256
    assert L.reax_fmha_splitkv_workspace(16, 8, 4, 128, 16) == want
    assert L.reax_fmha_splitkv_workspace(16, 8, 4, 64, 16) == 0  # unsupported head_dim
    assert L.reax_fmha_splitkv_workspace(16, 8, 4, 128, 0) == 0


def test_gemm_config_names_cover_the_tiles():
    # every index names one of the gfx950 tiles; index 0 is the 256 x 256 ring tile in each library (plain and slices
    # take the 256 x 160 one instead where that fills the CUs better), and every tile is reachable from some index of
    # each library (so a caller that times all indices tries each tile)
    P, S, G = abi.plain(), abi.slices(), abi.gv()
    for name, fn, n in (("plain", P.reax_gemm_cfgname, 15), ("slices", S.reax_slices_cfgname, 16),
                        ("gv", G.reax_gv_cfgname, 20)):
        names = [fn(c).decode() for c in range(n)]
        assert all(x.startswith("mfma ") for x in names), (name, names)
        assert names[0].startswith("mfma 256x256x64"), (name, names[0])
        assert len(set(names)) == 5, (name, sorted(set(names)))


def prototypes(header):
    """name -> (return type, argument declarations) of every function the header declares."""
    text = open(os.path.join(INC, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"^\s*((?:const\s+)?(?:int|size_t|char|void)\s*\*?)\s*(\w+)\s*\(([^;]*?)\)\s*;", text,
                         flags=re.M | re.S):
        args = m.group(3).strip()
        out[m.group(2)] = (re.sub(r"\s+", " ", m.group(1).strip()),
                           [] if args in ("", "void") else [re.sub(r"\s+", " ", a.strip()) for a in args.split(",")])
    return out


def c_to_ctypes(decl):
    """The ctypes type the loader must bind for one C argument declaration (every pointer and the stream: c_void_p)."""
    if "*" in decl or decl.startswith("hipStream_t"):
        return ctypes.c_void_p
    base = re.sub(r"\s\w+$", "", decl)  # the type without the argument's name
    return {"int": ctypes.c_int, "long long": ctypes.c_longlong, "float": ctypes.c_float,
            "size_t": ctypes.c_size_t}[base]


@pytest.mark.parametrize("header", sorted(h for h in os.listdir(INC) if h.endswith(".h")))
def test_binding_argtypes_match_prototypes(header):
    # the ctypes binding (abi.SIGNATURES / abi.RESTYPES) against the C prototypes, argument by argument: a count or
    # width mismatch would shift every later argument of the call
    protos = prototypes(header)
    assert protos, f"no prototypes parsed from {header}"
    assert set(declared(header)) <= set(protos), "a prototype the parser missed"
    for name, (ret, args) in protos.items():
        assert abi.SIGNATURES[name] == [c_to_ctypes(a) for a in args], name
        want_ret = {"int": None, "size_t": ctypes.c_size_t, "const char*": ctypes.c_char_p}[ret]
        assert abi.RESTYPES.get(name) == want_ret, name


def test_integration_doc_argtypes_match_binding():
    # INTEGRATION.md shows the loader's argtypes lines for a maintainer to copy: each must equal the binding's
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    names = {"P": ctypes.c_void_p, "I": ctypes.c_int, "LL": ctypes.c_longlong, "F": ctypes.c_float, "ctypes": ctypes}
    lines = re.findall(r"^\w+\.(\w+)\.argtypes = (.+)$", text, flags=re.M)
    assert len(lines) >= 10
    for name, expr in lines:
        assert eval(expr, {"__builtins__": {}}, names) == abi.SIGNATURES[name], name
