"""GPU parity of the GEMM libraries (libreax_plain.so, libreax_slices.so, libreax_gv.so; reference
libreax_plain/gemm_plain2.cu, libreax_slices/gemm_slices_v2.cu, libreax_gv/gateup_vis2.cu) through the C ABI against
float64 products of the same bf16 inputs: bf16 outputs within one bf16 ulp of the exactly rounded product plus
2^-14 of the output scale (fp32 accumulation in the library's order; the reference's own ascending-K fp32 order
gives its own last-bit pattern, so bit parity with it is not claimed), fp32 partials within 2^-18 of the scale; the
gate/up epilogue bf16(bf16(silu(bf16 g)) * bf16 u) against float64 SiLU of the bf16-rounded exact products, two
bf16 ulps."""
import numpy as np
import pytest

from reax_fmha import workloads as W
from rarn_cases import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _say(msg):
    print(f"[gpu-gemm] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _rand(shape, seed, scale=1.0):
    return f32_to_bf16((np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32))


def _close(got, ref, ulps, floor_rel):
    scale = np.abs(ref).max()
    bad = np.abs(got - ref) > np.abs(ref) * (ulps * 2.0 ** -8) + scale * floor_rel
    return int(bad.sum()), float(np.abs(got - ref).max() / scale)


@pytest.mark.parametrize("M,N,K,ldd,cfg", [(64, 64, 64, 64, 0), (300, 520, 1024, 520, 7), (8, 4096, 2560, 4104, 14),
                                           (1000, 136, 8, 144, 3), (1, 8, 8, 8, 2), (1, 8, 8, 8, 0),
                                           (257, 264, 8200, 264, 1)])
def test_plain_gemm(M, N, K, ldd, cfg):
    from reax_fmha import abi

    _say(f"plain M={M} N={N} K={K} ldd={ldd} cfg={cfg}")
    x, w = _rand((M, K), 1), _rand((N, K), 2)
    ref = bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(w).astype(np.float64).T
    dx, dw = W.bits_to_torch(x, "cuda"), W.bits_to_torch(w, "cuda")
    d = torch.full((M, ldd), float("nan"), dtype=torch.bfloat16, device="cuda")
    rc = abi.plain().reax_gemm(cfg, dx.data_ptr(), dw.data_ptr(), d.data_ptr(), M, N, K, ldd,
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    db = W.torch_to_bits(d).reshape(M, ldd)
    assert np.isnan(bf16_to_f32(db[:, N:])).all(), "wrote past column N"
    bad, rel = _close(bf16_to_f32(db[:, :N]).astype(np.float64), ref, 1, 2.0 ** -14)
    assert bad == 0, f"{bad} outputs off (max error {rel:.3g} of the scale)"


@pytest.mark.parametrize("K", [392, 512])
@pytest.mark.parametrize("lib", ["plain", "slices", "gv"])
def test_configs_bit_identical(lib, K):
    """Every config index (tile shape) adds each output's K terms in the same order: identical bits (the reference's
    configs share one reduction order too, gemm_slices_v2.cu:5-8)."""
    from reax_fmha import abi

    M, N = 300, 264  # K = 512: whole 64-deep slices, so the direct-to-LDS tiles run too
    x, w = _rand((M, K), 7), _rand((N, K), 8, 0.1)
    dx, dw = W.bits_to_torch(x, "cuda"), W.bits_to_torch(w, "cuda")
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    ncfg = {"plain": 15, "slices": 16, "gv": 20}[lib]
    for cfg in range(ncfg):
        _say(f"{lib} K={K} cfg={cfg}")
        if lib == "plain":
            o = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
            rc = abi.plain().reax_gemm(cfg, dx.data_ptr(), dw.data_ptr(), o.data_ptr(), M, N, K, N, st)
        elif lib == "slices":
            o = torch.zeros((2, M, N), dtype=torch.float32, device="cuda")
            rc = abi.slices().reax_slices(cfg, 1, dx.data_ptr(), dw.data_ptr(), o.data_ptr(), M, N, 192, 2, K, st)
        else:
            o = torch.zeros((M, N // 2), dtype=torch.bfloat16, device="cuda")
            rc = abi.gv().reax_gv(cfg, dx.data_ptr(), dw.data_ptr(), o.data_ptr(), M, N // 2, K, st)
        torch.cuda.synchronize()
        assert rc == 0
        outs.append(o.view(torch.int16 if o.dtype == torch.bfloat16 else torch.int32).cpu().numpy())
    for cfg in range(1, ncfg):
        assert np.array_equal(outs[cfg], outs[0]), f"config {cfg} differs from config 0"


@pytest.mark.parametrize("part_fp32", [1, 0])
@pytest.mark.parametrize("M,N,kps,S,K", [(64, 128, 256, 4, 1024), (200, 72, 64, 3, 200), (64, 128, 64, 2, 128),
                                          (130, 256, 520, 1, 520), (1, 8, 8, 1, 8), (33, 40, 8, 16, 128)])
def test_slices(M, N, kps, S, K, part_fp32):
    from reax_fmha import abi

    _say(f"slices M={M} N={N} kps={kps} S={S} K={K} fp32={part_fp32}")
    x, w = _rand((M, K), 3), _rand((N, K), 4)
    xf, wf = bf16_to_f32(x).astype(np.float64), bf16_to_f32(w).astype(np.float64)
    dt = torch.float32 if part_fp32 else torch.bfloat16
    p = torch.zeros((S, M, N), dtype=dt, device="cuda")
    dx, dw = W.bits_to_torch(x, "cuda"), W.bits_to_torch(w, "cuda")  # held: a freed temporary's block is reused
    rc = abi.slices().reax_slices(kps // 8 % 4, part_fp32, dx.data_ptr(), dw.data_ptr(), p.data_ptr(), M, N, kps, S, K,
                                  torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    for s in range(S):
        ref = xf[:, s * kps:(s + 1) * kps] @ wf[:, s * kps:(s + 1) * kps].T
        got = p[s].float().cpu().numpy().astype(np.float64)
        bad, rel = _close(got, ref, 0 if part_fp32 else 1, 2.0 ** -18 if part_fp32 else 2.0 ** -14)
        assert bad == 0, f"slice {s}: {bad} partials off (max error {rel:.3g} of the scale)"


@pytest.mark.parametrize("M,N2,K,cfg", [(128, 64, 256, 0), (77, 100, 520, 1), (512, 1024, 2560, 2), (300, 260, 64, 3),
                                        (130, 516, 136, 0), (1, 4, 8, 2), (1, 4, 8, 16), (513, 132, 4104, 16)])
def test_gv(M, N2, K, cfg):
    from reax_fmha import abi

    _say(f"gv M={M} N2={N2} K={K} cfg={cfg}")
    x, w = _rand((M, K), 5, 0.5), _rand((2 * N2, K), 6, 0.05)
    c = bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(w).astype(np.float64).T      # [M][2 N2]
    cg = c.reshape(M, N2 // 4, 2, 4)
    g = bf16_to_f32(f32_to_bf16(cg[:, :, 0].astype(np.float32))).astype(np.float64)
    u = bf16_to_f32(f32_to_bf16(cg[:, :, 1].astype(np.float32))).astype(np.float64)
    s = bf16_to_f32(f32_to_bf16((g / (1.0 + np.exp(-g))).astype(np.float32))).astype(np.float64)
    ref = (s * u).reshape(M, N2)
    out = torch.full((M, N2), float("nan"), dtype=torch.bfloat16, device="cuda")
    dx, dw = W.bits_to_torch(x, "cuda"), W.bits_to_torch(w, "cuda")
    rc = abi.gv().reax_gv(cfg, dx.data_ptr(), dw.data_ptr(), out.data_ptr(), M, N2, K,
                          torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    got = out.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all(), "an activation left unwritten"
    bad, rel = _close(got, ref, 2, 2.0 ** -12)
    assert bad == 0, f"{bad} activations off (max error {rel:.3g} of the scale)"


@pytest.mark.parametrize("lib", ["plain", "gv"])
def test_offset_bases(lib):
    """X and W starting 16 bytes into their allocations (the ABI asks for 16-byte alignment only): same bits as the
    aligned call, on a whole-slice K (the direct-to-LDS tiles) and a ragged one (register-staged)."""
    from reax_fmha import abi

    st = torch.cuda.current_stream().cuda_stream
    for K in (512, 200):
        M, N = 136, 264
        _say(f"{lib} offset bases K={K}")
        x, w = _rand((M, K), 11), _rand((N, K), 12, 0.1)
        dx, dw = W.bits_to_torch(x, "cuda"), W.bits_to_torch(w, "cuda")
        bx = torch.zeros(M * K + 8, dtype=torch.bfloat16, device="cuda")
        bw = torch.zeros(N * K + 8, dtype=torch.bfloat16, device="cuda")
        bx[8:] = dx.reshape(-1)
        bw[8:] = dw.reshape(-1)
        outs = []
        for px, pw in ((dx.data_ptr(), dw.data_ptr()), (bx.data_ptr() + 16, bw.data_ptr() + 16)):
            if lib == "plain":
                o = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
                rc = abi.plain().reax_gemm(0, px, pw, o.data_ptr(), M, N, K, N, st)
            else:
                o = torch.zeros((M, N // 2), dtype=torch.bfloat16, device="cuda")
                rc = abi.gv().reax_gv(0, px, pw, o.data_ptr(), M, N // 2, K, st)
            torch.cuda.synchronize()
            assert rc == 0
            outs.append(o.view(torch.int16).cpu().numpy())
        assert np.array_equal(outs[0], outs[1]), f"K={K}: offset bases change the result"
