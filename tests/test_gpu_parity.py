"""GPU parity: the HIP kernels, called through the C ABI, against the double-precision CPU oracle (and the
golden fixtures), to the tolerance of the path: bf16 outputs max-abs <= 2e-2 and mean-abs <= 2e-3, LSE within
1e-3 relative (|dLSE| <= 1e-3 * |LSE| + 1e-5). Large configurations are checked on a seeded subset of tokens
(first and last tokens plus random ones; rows are independent) with every head."""
import glob
import os

import numpy as np
import pytest

import fmha_cases as FC
import pyoracle
from reax_fmha import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _say(msg):
    print(f"[gpu-parity] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from reax_fmha import abi

    abi.howu()
    abi.post()


def dev(bits):
    return W.bits_to_torch(bits, "cuda")


def host(t):
    return W.torch_to_bits(t)


def run_qx(c: FC.Case, a: dict, want_lse=True):
    from reax_fmha import ops

    q, k, v = dev(a["q"]), dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(a["qpos"]).cuda()
    o, lse = ops.attention(q, k, v, qpos, scale=c.scale, want_lse=want_lse)
    torch.cuda.synchronize()
    return host(o), (lse.cpu().numpy() if lse is not None else None)


def token_subset(S, n_rand, seed, edge=64):
    rng = np.random.default_rng(seed)
    sel = set(range(min(edge, S))) | set(range(max(0, S - edge), S))
    sel |= set(int(x) for x in rng.integers(0, S, size=n_rand))
    return np.array(sorted(sel), dtype=np.int64)


def torch_causal_check(og_bits, lg, q_bits, k_bits, v_bits, G, scale, *, gate_bits=None, chunk=1024, where=""):
    """Every row of a B = 1 causal attention (N == S) against a float32 torch reference on the GPU, row chunk by row
    chunk, to the parity bar of check_tolerance: the full-size complement of the oracle's seeded token subset.
    og_bits is the kernel's bf16 output [S][Hq][D] (bits), lg its LSE [Hq][S] or None. With gate_bits [S][Hq][D]
    the reference is the POST output O * sigmoid(gate). Float32 matmuls on contiguous operands only."""
    q = dev(q_bits)[0].float()
    S, Hq, D = q.shape
    kt = dev(k_bits)[0].float().permute(1, 2, 0).repeat_interleave(G, 0).contiguous()  # [Hq][D][N]
    vh = dev(v_bits)[0].float().permute(1, 0, 2).repeat_interleave(G, 0).contiguous()  # [Hq][N][D]
    og = dev(og_bits).reshape(S, Hq, D)
    gate = dev(gate_bits).reshape(S, Hq, D) if gate_bits is not None else None
    lgd = torch.from_numpy(np.ascontiguousarray(lg)).to(q.device).reshape(Hq, S) if lg is not None else None
    worst, tot, lworst = 0.0, 0.0, 0.0
    for r0 in range(0, S, chunk):
        r1 = min(S, r0 + chunk)
        s = torch.matmul(q[r0:r1].permute(1, 0, 2).contiguous(), kt[:, :, :r1].contiguous()).mul_(scale)
        rows = torch.arange(r0, r1, device=q.device)[:, None]
        s.masked_fill_(torch.arange(r1, device=q.device)[None, :] > rows, float("-inf"))
        lse = torch.logsumexp(s, dim=-1)  # [Hq][R]
        o = torch.matmul(s.sub_(lse[..., None]).exp_(), vh[:, :r1].contiguous()).permute(1, 0, 2)  # [R][Hq][D]
        del s
        if gate is not None:
            o = o * torch.sigmoid(gate[r0:r1].float())
        got = og[r0:r1].float()
        assert torch.isfinite(got).all(), f"{where}: non-finite output in rows {r0}..{r1}"
        err = (got - o).abs_()
        worst = max(worst, float(err.max()))
        tot += float(err.double().sum())
        if lgd is not None:
            d = (lgd[:, r0:r1] - lse).abs_()
            excess = float((d - (1e-3 * lse.abs() + 1e-5)).max())
            assert excess <= 0, f"{where}: LSE beyond 1e-3 relative in rows {r0}..{r1}"
            lworst = max(lworst, float((d / (lse.abs() + 1e-2)).max()))
    mean = tot / (S * Hq * D)
    assert worst <= 2e-2, f"{where}: max-abs {worst:.3g} > 2e-2 (all rows, float32 reference)"
    assert mean <= 2e-3, f"{where}: mean-abs {mean:.3g} > 2e-3 (all rows, float32 reference)"
    return dict(max_abs=worst, mean_abs=mean, lse_rel=lworst)


def oracle_on_tokens(c: FC.Case, a: dict, toks):
    """Oracle rows for the given query tokens only (qpos keeps each token's own visibility)."""
    sub = FC.Case(c.name + "_sub", B=c.B, S=len(toks), N=c.N, Hq=c.Hq, Hkv=c.Hkv, D=c.D, mode="qpos",
                  qpos=a["qpos"][:, toks])
    asub = dict(q=np.ascontiguousarray(a["q"][:, toks]), k=a["k"], v=a["v"], qpos=sub.qpos)
    return FC.oracle_ref(sub, asub)


# ------------------------------------------------------------------------------------------ qx (extension ABI)

SMALL = [
    FC.Case("c1_shape", B=1, S=512, N=512, Hq=8, Hkv=2, D=128, mode="causal", seed=1001),
    FC.Case("ragged_s77_g4", B=2, S=77, N=77, Hq=8, Hkv=2, D=128, mode="causal", seed=3),
    FC.Case("prefix_s50_n333", B=1, S=50, N=333, Hq=4, Hkv=4, D=128, mode="causal", seed=4),
    FC.Case("g8_s200_d128", B=1, S=200, N=200, Hq=8, Hkv=1, D=128, mode="causal", seed=5),
    FC.Case("full_s3_n1000", B=3, S=3, N=1000, Hq=8, Hkv=2, D=128, mode="full", seed=6),
    FC.Case("d256_s300_g2", B=1, S=300, N=300, Hq=4, Hkv=2, D=256, mode="causal", seed=7),
    FC.Case("d256_full_n129", B=2, S=17, N=129, Hq=2, Hkv=1, D=256, mode="full", seed=8),
    FC.Case("n1_single_key", B=1, S=5, N=1, Hq=4, Hkv=2, D=128, mode="full", seed=9),
    # enough (b, KV head) row tiles for the ping-pong kernel (the shapes above take the row-block kernel)
    FC.Case("pp_ragged_s77_b9", B=9, S=77, N=77, Hq=32, Hkv=8, D=128, mode="causal", seed=10),
    FC.Case("pp_prefix_s50_n333", B=9, S=50, N=333, Hq=32, Hkv=8, D=128, mode="causal", seed=11),
    # at most 128 folded rows with too many (b, KV head) pairs for the row-block kernel: the 4-wavefront kernel
    FC.Case("fwd4_s20_b9", B=9, S=20, N=20, Hq=32, Hkv=8, D=128, mode="causal", seed=12),
    FC.Case("fwd4_s5_n700_b9", B=9, S=5, N=700, Hq=32, Hkv=8, D=128, mode="causal", seed=13),
]


def qx_route(c: FC.Case) -> str:
    """The head_dim-128 qx kernel a shape reaches: the row-block kernel when the ping-pong kernel's 256-row items
    would occupy at most a quarter of the CUs, else the ping-pong kernel (more than 128 folded rows) or the
    4-wavefront kernel (128 rows a workgroup)."""
    M = c.S * c.G
    items = c.B * c.Hkv * -(-M // 256)
    if c.D == 128 and items * 4 <= torch.cuda.get_device_properties(0).multi_processor_count:
        return "rows"
    return "pp" if M > 128 else "fwd4"


@pytest.mark.parametrize("c", SMALL, ids=lambda c: c.name)
def test_qx_against_oracle(c):
    _say(f"qx {c.name} B{c.B} S{c.S} N{c.N} Hq{c.Hq} Hkv{c.Hkv} D{c.D} ({qx_route(c)} kernel)")
    a = FC.build(c)
    og, lg = run_qx(c, a)
    o, lse = FC.oracle_ref(c, a)
    res = FC.check_tolerance(og, o, lg, lse, where=c.name)
    _say(f"  {res}")


@pytest.mark.parametrize("B,Hq,Hkv,route", [(1, 8, 2, "rows"), (9, 32, 8, "pp")], ids=["rows", "pp"])
def test_qx_qpos_edges(B, Hq, Hkv, route):
    """qpos < 0 rows give 0 / -inf; qpos = 0 rows reproduce V[0] exactly; qpos >= N sees every key; rows in any
    order (qpos not increasing), on both head_dim-128 prefill kernels."""
    S, N = 40, 150
    rng = np.random.default_rng(21)
    qp = rng.integers(-2, N + 4, size=(B, S)).astype(np.int32)
    qp[:, :4] = [0, -1, N + 3, 63]
    c = FC.Case(f"qpos_edges_{route}", B=B, S=S, N=N, Hq=Hq, Hkv=Hkv, D=128, mode="qpos", seed=22, qpos=qp)
    assert qx_route(c) == route
    _say(f"qx {c.name}")
    a = FC.build(c)
    og, lg = run_qx(c, a)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where=c.name)
    for b in range(B):
        dead = qp[b] < 0
        assert (og[b, dead] == 0).all() and np.isneginf(lg[b][:, dead]).all()
        for m in np.nonzero(qp[b] == 0)[0]:
            for hq in range(c.Hq):
                assert (og[b, m, hq] == a["v"][b, 0, hq // c.G]).all(), "qpos = 0 must write V[0] exactly"


# The head_dim-128 prefill kernel is persistent (one workgroup per CU, items in snake order, an XCD-aware split
# when B*H % 8 == 0): these shapes give more items than CUs, so workgroups run several items, in both orders.
@pytest.mark.parametrize("B,S,Hq,Hkv", [(2, 2304, 16, 8), (1, 11264, 6, 3)], ids=["xcd_split", "plain_order"])
def test_qx_persistent_multi_item(B, S, Hq, Hkv):
    c = FC.Case(f"persist_b{B}_s{S}", B=B, S=S, N=S, Hq=Hq, Hkv=Hkv, D=128, mode="causal", seed=23 + B)
    _say(f"qx persistent B{B} S{S} Hq{Hq} Hkv{Hkv} ({B * Hkv * -(-S * (Hq // Hkv) // 256)} items)")
    a = FC.build(c)
    og, lg = run_qx(c, a)
    toks = token_subset(S, 48, 31 + B, edge=32)
    o, lse = oracle_on_tokens(c, a, toks)
    FC.check_tolerance(og[:, toks], o, lg[:, :, toks], lse, where=c.name)
    assert np.isfinite(W.bf16_bits_to_f32(og)).all()


# The head_dim-128 prefill kernel picks its output store by the output's alignment: rows 16-byte aligned go out as
# whole rows staged through LDS, 8-byte aligned ones as 8-byte pieces, the rest as 4-byte pieces. An output view
# into rows padded by `pad` elements selects each; the padding must stay untouched.
# The row-block kernel stores 16 bytes per thread when the output's rows are 16-byte aligned, else 4-byte pieces.
@pytest.mark.parametrize("pad", [8, 4, 2], ids=["rows16", "rows8", "rows4"])
@pytest.mark.parametrize("B,Hq,Hkv,route", [(2, 8, 2, "rows"), (9, 32, 8, "pp")], ids=["rows", "pp"])
def test_qx_output_strides(pad, B, Hq, Hkv, route):
    from reax_fmha import ops

    c = FC.Case(f"ostride_pad{pad}_{route}", B=B, S=120, N=120, Hq=Hq, Hkv=Hkv, D=128, mode="causal", seed=41 + pad)
    assert qx_route(c) == route
    _say(f"qx output rows padded by {pad} ({route} kernel)")
    a = FC.build(c)
    q, k, v = dev(a["q"]), dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(a["qpos"]).cuda()
    buf = torch.full((c.B, c.S, c.Hq, c.D + pad), -7.0, dtype=torch.bfloat16, device="cuda")
    o = buf[..., : c.D]
    _, lse = ops.attention(q, k, v, qpos, scale=c.scale, o=o)
    torch.cuda.synchronize()
    assert (buf[..., c.D:] == -7.0).all(), "padding written"
    o_ref, lse_ref = FC.oracle_ref(c, a)
    FC.check_tolerance(host(o.contiguous()), o_ref, lse.cpu().numpy(), lse_ref, where=c.name)


# The row-block kernel (head_dim-128 prefills too small to fill the GPU with 256-row items): 32-row blocks, the
# block's 32-key tiles dealt to 8 wavefronts (tiles w, w + 8, ...), merged in LDS. Partial last blocks, fewer rows
# than a block, G = 1 and 16, key ranges of one tile to 129 tiles (a partial last tile; up to 17 tiles per
# wavefront), wavefronts left without a tile (a block seeing fewer tiles than there are wavefronts), random qpos
# with negatives and qpos >= N, and no LSE output.
ROWS = [
    FC.Case("rows_ragged_b3_s77", B=3, S=77, N=77, Hq=8, Hkv=2, D=128, mode="causal", seed=51),
    FC.Case("rows_m24_n4100", B=2, S=3, N=4100, Hq=16, Hkv=2, D=128, mode="full", seed=52),
    FC.Case("rows_g1_s33_n600", B=1, S=33, N=600, Hq=4, Hkv=4, D=128, mode="causal", seed=53),
    FC.Case("rows_g16_s130", B=1, S=130, N=130, Hq=16, Hkv=1, D=128, mode="causal", seed=54),
    FC.Case("rows_qpos_rand", B=2, S=61, N=300, Hq=8, Hkv=2, D=128, mode="qpos", seed=55,
            qpos=np.random.default_rng(56).integers(-3, 306, size=(2, 61)).astype(np.int32)),
    FC.Case("rows_n65", B=1, S=9, N=65, Hq=8, Hkv=8, D=128, mode="full", seed=57),
]


@pytest.mark.parametrize("c", ROWS, ids=lambda c: c.name)
@pytest.mark.parametrize("want_lse", [True, False], ids=["lse", "no_lse"])
def test_qx_rows_kernel(c, want_lse):
    assert qx_route(c) == "rows"
    _say(f"qx rows {c.name} B{c.B} S{c.S} N{c.N} Hq{c.Hq} Hkv{c.Hkv} lse={want_lse}")
    a = FC.build(c)
    og, lg = run_qx(c, a, want_lse=want_lse)
    o, lse = FC.oracle_ref(c, a)
    res = FC.check_tolerance(og, o, lg, lse if want_lse else None, where=c.name)
    _say(f"  {res}")


# The routing bound: 64 ping-pong items on 256 CUs (a quarter) take the row-block kernel (512 workgroups, two per
# CU in turn), 72 take the ping-pong kernel; both checked on a seeded token subset.
@pytest.mark.parametrize("S,route", [(512, "rows"), (520, "pp")], ids=["rows_64_items", "pp_72_items"])
def test_qx_route_bound(S, route):
    c = FC.Case(f"route_s{S}", B=1, S=S, N=S, Hq=32, Hkv=8, D=128, mode="causal", seed=60 + S)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the bound is placed for 256 CUs")
    assert qx_route(c) == route
    _say(f"qx {c.name} ({route} kernel)")
    a = FC.build(c)
    og, lg = run_qx(c, a)
    toks = token_subset(S, 40, 61, edge=24)
    o, lse = oracle_on_tokens(c, a, toks)
    FC.check_tolerance(og[:, toks], o, lg[:, :, toks], lse, where=c.name)


def _random_rows_cases(n, seed):
    """Seeded random shapes for the row-block kernel: B 1-3, Hkv 1-4, G 1/2/4/8/16, S 1-300 tokens, N 1-1200 keys,
    causal, full or random qpos (negatives and qpos >= N included), each kept within the row-block bound
    (B * Hkv * ceil(S * G / 256) <= 64) and small enough for the double-precision oracle."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B, Hkv, G = int(rng.integers(1, 4)), int(rng.integers(1, 5)), int(rng.choice([1, 2, 4, 8, 16]))
        S, N = int(rng.integers(1, 301)), int(rng.integers(1, 1201))
        if B * Hkv * -(-S * G // 256) > 64 or B * S * Hkv * G * N > 6_000_000:
            continue
        mode = str(rng.choice(["causal", "full", "qpos"]))
        if mode == "causal" and N < S:
            N = S
        qp = rng.integers(-3, N + 3, size=(B, S)).astype(np.int32) if mode == "qpos" else None
        out.append(FC.Case(f"rand{len(out)}_b{B}_h{Hkv}_g{G}_s{S}_n{N}_{mode}", B=B, S=S, N=N, Hq=Hkv * G, Hkv=Hkv,
                           D=128, mode=mode, seed=int(rng.integers(1 << 30)), qpos=qp))
    return out


# Random shapes through the row-block kernel against the oracle (a sweep on top of the hand-picked cases above).
@pytest.mark.parametrize("c", _random_rows_cases(24, 2026), ids=lambda c: c.name)
def test_qx_rows_random(c):
    assert qx_route(c) == "rows"
    _say(f"qx rows random {c.name}")
    a = FC.build(c)
    og, lg = run_qx(c, a)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where=c.name)


GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p))
def test_golden(path):
    import golden_io

    c, a, o_want, lse_want = golden_io.load(path)
    _say(f"golden {c.name}")
    if c.mode == "bias":
        og = run_bias(c, a)
        FC.check_tolerance(og, o_want, where=c.name)
    else:
        og, lg = run_qx(c, a)
        FC.check_tolerance(og, o_want, lg, lse_want, where=c.name)
        if c.S == 1:  # a decode fixture: the split-KV path too, with one, several and more splits than key tiles
            for n in (1, 3, 16):
                og, lg = run_split(c, a, n)
                FC.check_tolerance(og, o_want, lg, lse_want, where=f"{c.name} split{n}")


# ------------------------------------------------------------------------------------------ drop-in ABI

def fold(x, G):
    """natural [B][S][Hq][D] -> folded [B][Hkv][S*G][D] (row r = m*G + g)."""
    B, S, Hq, D = x.shape
    return np.ascontiguousarray(x.reshape(B, S, Hq // G, G, D).transpose(0, 2, 1, 3, 4).reshape(B, Hq // G, S * G, D))


def unfold(x, G):
    B, H, M, D = x.shape
    S = M // G
    return x.reshape(B, H, S, G, D).transpose(0, 2, 1, 3, 4).reshape(B, S, H * G, D)


@pytest.mark.parametrize("lib", ["howu", "post"])
@pytest.mark.parametrize("S,G,Hkv", [(64, 8, 2), (45, 4, 1), (130, 1, 2)])
def test_reax_fmha_q_dropin(lib, S, G, Hkv):
    from reax_fmha import ops

    c = FC.Case(f"q_{lib}_{S}_{G}", B=2, S=S, N=S, Hq=G * Hkv, Hkv=Hkv, D=256, mode="causal", seed=30 + S)
    _say(f"reax_fmha_q {lib} S{S} G{G} Hkv{Hkv}")
    a = FC.build(c)
    q = dev(fold(a["q"], G))
    k, v = dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(a["qpos"]).cuda()
    o = torch.full_like(q, float("nan"))
    ops.fmha_q(q, k, v, qpos, G, o, c.scale, lib=lib)
    torch.cuda.synchronize()
    og = unfold(host(o), G)
    oref, _ = FC.oracle_ref(c, a)
    FC.check_tolerance(og, oref, where=c.name)


def _block_rule_cases():
    """qpos patterns for the drop-in block-wide qpos = 0 rule (64 folded rows per block, reax_fmha_v8.cu:155-162,
    224-235): G = 8 blocks {0, -1 x 7}, {-1 x 8}, {0, 0, -1, ...}, {5, -1, 0, ...} (per-row), {-1 ..., 0}; G = 3,
    where token 21's rows straddle two blocks."""
    qp8 = np.array([0] + [-1] * 7 + [-1] * 8 + [0, 0] + [-1] * 6 + [5, -1, 0] + [-1] * 5 + [-1] * 7 + [0],
                   dtype=np.int32)
    qp3 = np.full(30, -1, dtype=np.int32)
    qp3[5], qp3[25] = 0, 2
    return [FC.Case("blk_g8", B=1, S=40, N=50, Hq=16, Hkv=2, D=256, mode="qpos", seed=35, qpos=qp8[None]),
            FC.Case("blk_g3", B=1, S=30, N=20, Hq=3, Hkv=1, D=256, mode="qpos", seed=36, qpos=qp3[None])]


def _v0_rows(c, a):
    """(token, query head) pairs that the drop-in rule stores as V[0]: rows of blocks whose largest qpos is 0."""
    out = []
    qp = a["qpos"][0]
    M = c.S * c.G
    for j in range(0, M, 64):
        rows = range(j, min(j + 64, M))
        if max(int(qp[r // c.G]) for r in rows) == 0:
            for h in range(c.Hkv):
                out += [(r // c.G, h * c.G + r % c.G) for r in rows]
    return out


@pytest.mark.parametrize("lib", ["howu", "post"])
@pytest.mark.parametrize("ci", [0, 1], ids=["g8", "g3"])
def test_reax_fmha_q_qpos0_block(lib, ci):
    """reax_fmha_q applies the reference's block-wide qpos = 0 shortcut: GPU = oracle (drop-in mode) = V[0]
    bit for bit on every row of a block whose largest qpos is 0, qpos < 0 rows included."""
    from reax_fmha import ops

    c = _block_rule_cases()[ci]
    _say(f"reax_fmha_q qpos0 block {lib} {c.name}")
    a = FC.build(c)
    G = c.G
    q = dev(fold(a["q"], G))
    k, v = dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(a["qpos"]).cuda()
    o = torch.full_like(q, float("nan"))
    ops.fmha_q(q, k, v, qpos, G, o, c.scale, lib=lib)
    torch.cuda.synchronize()
    og = unfold(host(o), G)
    oref, _ = FC.oracle_ref(c, a, dropin=True)
    FC.check_tolerance(og, oref, where=c.name)
    v0 = _v0_rows(c, a)
    assert v0, "the case must contain a block whose largest qpos is 0"
    for m, hq in v0:
        assert (og[0, m, hq] == a["v"][0, 0, hq // G]).all(), f"token {m} head {hq}: V[0] expected"
        assert (oref[0, m, hq] == W.bf16_bits_to_f32(a["v"][0, 0, hq // G])).all()
    dead = [(m, hq) for m in range(c.S) for hq in range(c.Hq) if a["qpos"][0, m] < 0 and (m, hq) not in set(v0)]
    for m, hq in dead:
        assert (og[0, m, hq] == 0).all(), f"token {m} head {hq}: 0 expected"


def test_reax_fmha_qp_qpos0_block():
    """The POST path of the block rule: rows of a block whose largest qpos is 0 gate V[0]."""
    c = _block_rule_cases()[0]
    _say("reax_fmha_qp qpos0 block")
    a = FC.build(c)
    rng = np.random.default_rng(37)
    T = c.S
    inv = np.arange(T, dtype=np.int32)
    qg = W.bf16_normal(rng, (T, c.Hq, 2 * c.D))
    got = run_post(c, a, qg, inv, T)
    o, _ = FC.oracle_ref(c, a, dropin=True)
    want = np.full((T, c.Hq * c.D), 0x7E00, dtype=np.uint16)
    pyoracle.post_gate(fold_dense(o, c.G), B=1, H=c.Hkv, G=c.G, M=c.S * c.G, D=c.D, inv=inv, Lq=c.S, qg=qg,
                       qg_rs=c.Hq * 2 * c.D, out=want, out_rs=c.Hq * c.D)
    for m, hq in _v0_rows(c, a):
        sl = slice(hq * c.D, (hq + 1) * c.D)
        assert (got[m, sl] == want[m, sl]).all(), f"token {m} head {hq}: gated V[0] expected bit for bit"
    FC.check_tolerance(got, W.bf16_bits_to_f32(want).astype(np.float64), where="qp block rule")


def run_bias(c, a, lib="howu"):
    from reax_fmha import ops

    q = dev(fold(a["q"], 1))
    k, v = dev(a["k"]), dev(a["v"])
    bias = dev(a["bias"])
    o = torch.full_like(q, float("nan"))
    ops.fmha_b(q, k, v, bias, o, c.scale, lib=lib)
    torch.cuda.synchronize()
    return unfold(host(o), 1)


@pytest.mark.parametrize("lib", ["howu", "post"])
def test_reax_fmha_b(lib):
    c = FC.Case("bias", B=2, S=70, N=150, Hq=2, Hkv=2, D=256, mode="bias", seed=41, bias_neg_inf_frac=0.2,
                bias_full_rows=(5, 69))
    _say(f"reax_fmha_b {lib}")
    a = FC.build(c)
    og = run_bias(c, a, lib)
    oref, _ = FC.oracle_ref(c, a)
    FC.check_tolerance(og, oref, where=c.name)
    assert (og[:, [5, 69]] == 0).all(), "an all -inf bias row must give 0"


def run_post(c, a, qg_bits, inv, T):
    from reax_fmha import ops

    G = c.G
    q = dev(fold(a["q"], G))
    k, v = dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(a["qpos"]).cuda()
    qg = dev(qg_bits)
    out = torch.from_numpy(np.full((T, c.Hq * c.D), 0x7E00, dtype=np.uint16).view(np.int16)).cuda().view(torch.bfloat16)
    invd = torch.from_numpy(inv).cuda()
    ops.fmha_qp(q, k, v, qpos, G, c.scale, invd, c.S, qg, out)
    torch.cuda.synchronize()
    return host(out)


def test_reax_fmha_qp_post():
    c = FC.Case("post", B=1, S=96, N=96, Hq=16, Hkv=2, D=256, mode="causal", seed=51)
    _say("reax_fmha_qp post S96")
    a = FC.build(c)
    rng = np.random.default_rng(52)
    T = c.S + 5
    inv = rng.permutation(T)[: c.S].astype(np.int32)
    inv[[3, 50]] = -1
    qg = W.bf16_normal(rng, (T, c.Hq, 2 * c.D))
    got = run_post(c, a, qg, inv, T)
    o, _ = FC.oracle_ref(c, a)
    want = np.full((T, c.Hq * c.D), 0x7E00, dtype=np.uint16)
    pyoracle.post_gate(fold_dense(o, c.G), B=1, H=c.Hkv, G=c.G, M=c.S * c.G, D=c.D, inv=inv, Lq=c.S, qg=qg,
                       qg_rs=c.Hq * 2 * c.D, out=want, out_rs=c.Hq * c.D)
    untouched = np.setdiff1d(np.arange(T), inv[inv >= 0])
    assert (got[untouched] == 0x7E00).all(), "rows not named by inv must stay untouched"
    rows = inv[inv >= 0]
    wf = W.bf16_bits_to_f32(want[rows]).astype(np.float64)
    FC.check_tolerance(got[rows], wf, where="post")


def fold_dense(o_nat, G):
    B, S, Hq, D = o_nat.shape
    return o_nat.reshape(B, S, Hq // G, G, D).transpose(0, 2, 1, 3, 4).reshape(B, Hq // G, S * G, D)


def test_post_sigmoid_exhaustive():
    """With V = 1 the attention output is exactly 1, so the POST output is the kernel's bf16 sigmoid of the gate:
    every one of the 65,536 bf16 gate values must give the correctly rounded sigmoid (bit-exact)."""
    S, G, Hkv, D = 16, 16, 1, 256
    c = FC.Case("sig", B=1, S=S, N=S, Hq=G * Hkv, Hkv=Hkv, D=D, mode="causal", seed=61)
    _say("post sigmoid exhaustive")
    a = FC.build(c)
    a["v"] = np.full_like(a["v"], 0x3F80)
    gates = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(S, G, D)
    qg = np.zeros((S, G, 2 * D), dtype=np.uint16)
    qg[:, :, D:] = gates
    inv = np.arange(S, dtype=np.int32)
    got = run_post(c, a, qg, inv, S).reshape(S, G, D)
    want = pyoracle.sigmoid_bf16_all()[gates]
    nan = np.isnan(W.bf16_bits_to_f32(want))
    assert np.isnan(W.bf16_bits_to_f32(got[nan])).all()
    bad = np.nonzero((got != want) & ~nan)
    assert bad[0].size == 0, f"{bad[0].size} sigmoid mismatches, e.g. gate {gates[bad][:4]} -> {got[bad][:4]} vs {want[bad][:4]}"


# ------------------------------------------------------------------------------------------ varlen

def run_varlen(c, a, want_lse=True):
    from reax_fmha import ops

    q, k, v = dev(a["q"]), dev(a["k"]), dev(a["v"])
    cu = torch.from_numpy(a["cu"]).cuda()
    o, lse = ops.attention_varlen(q, k, v, cu, max(c.seqlens), scale=c.scale, want_lse=want_lse)
    torch.cuda.synchronize()
    return host(o), (lse.cpu().numpy() if lse is not None else None)


# the third case keeps max_seqlen * G <= 128 (head_dim 128): the 4-wavefront kernel instead of the ping-pong one
@pytest.mark.parametrize("seqlens,D", [([5, 300, 0, 1, 129, 64], 128), ([200, 33, 97], 256), ([5, 30, 0, 1, 17, 32], 128)])
def test_varlen_ragged(seqlens, D):
    c = FC.Case("varlen", B=1, S=0, N=0, Hq=8, Hkv=2, D=D, mode="varlen", seed=71, seqlens=seqlens)
    _say(f"varlen {seqlens} D{D}")
    a = FC.build(c)
    og, lg = run_varlen(c, a)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where="varlen")


# Sequences of whole 256-row tiles (G = 4: 64 tokens a tile) in several sequences, so every wavefront of the
# prefill kernel reads its Q rows back from LDS with no row past a tile's end: a read that overtook the copies
# of its last rows showed up here as wrong rows 24..31 of the second wavefront group.
def test_varlen_full_tiles():
    c = FC.Case("varlen_full_tiles", B=1, S=0, N=0, Hq=8, Hkv=2, D=128, mode="varlen", seed=73,
                seqlens=[64, 64, 192, 128, 64, 320])
    _say(f"varlen full tiles {c.seqlens}")
    a = FC.build(c)
    og, lg = run_varlen(c, a)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where="varlen_full_tiles")


# The item schedule's other shapes: 96 sequences with 4 KV heads (48 pairs per class of 32 workgroups, ~100 items
# per class: six assignment rounds), 256 sequences with 8 KV heads (256 pairs per class: the pair table and its
# prefix sums over all 64 lanes of the scan) and 300 sequences (beyond its 256-sequence tables: the fixed order).
@pytest.mark.parametrize("nseq,hi,Hkv,seed", [(96, 400, 4, 75), (256, 200, 8, 77), (300, 24, 2, 76)])
def test_varlen_schedule_shapes(nseq, hi, Hkv, seed):
    seqlens = [int(x) for x in np.random.default_rng(seed).integers(0, hi, size=nseq)]
    c = FC.Case("varlen_sched", B=1, S=0, N=0, Hq=8, Hkv=Hkv, D=128, mode="varlen", seed=seed, seqlens=seqlens)
    _say(f"varlen schedule shapes nseq {nseq} Hkv {Hkv} tokens {sum(seqlens)}")
    a = FC.build(c)
    og, lg = run_varlen(c, a)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where=f"varlen_sched_{nseq}")


def test_config3_varlen():
    cfg = W.CONFIGS[3]
    c = FC.Case(cfg.name, B=1, S=0, N=0, Hq=cfg.Hq, Hkv=cfg.Hkv, D=cfg.D, mode="varlen", seed=cfg.seed,
                seqlens=cfg.seqlens)
    _say(f"config 3 varlen {cfg.seqlens}")
    q, k, v, cu = W.make_varlen_inputs(cfg)
    a = dict(q=q, k=k, v=v, cu=cu)
    og, lg = run_varlen(c, a)
    o, lse = FC.oracle_ref(c, a)
    res = FC.check_tolerance(og, o, lg, lse, where="config3")
    _say(f"  config 3 vs oracle (all rows): {res}")


# ------------------------------------------------------------------------------------------ split-KV decode

def run_split(c, a, num_splits):
    from reax_fmha import ops

    q, k, v = dev(a["q"]), dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(a["qpos"]).cuda()
    o, lse = ops.attention_splitkv(q, k, v, qpos, scale=c.scale, num_splits=num_splits)
    torch.cuda.synchronize()
    return host(o), lse.cpu().numpy()


@pytest.mark.parametrize("num_splits", [1, 3, 16, 40, 70])
def test_splitkv_small(num_splits):
    rng = np.random.default_rng(80)
    B, N = 3, 1000
    qp = np.array([[N - 1], [313], [-1]], dtype=np.int32)  # full cache, a shorter cache, an empty one
    c = FC.Case("split", B=B, S=1, N=N, Hq=8, Hkv=2, D=128, mode="qpos", seed=81, qpos=qp)
    _say(f"splitkv small S{num_splits}")
    a = FC.build(c)
    og, lg = run_split(c, a, num_splits)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where=f"split{num_splits}")
    assert (og[2] == 0).all() and np.isneginf(lg[2]).all()


@pytest.mark.parametrize("S,Hq,Hkv,N,splits", [(4, 32, 4, 2100, 7), (3, 8, 4, 70, 9), (1, 8, 8, 5000, 2),
                                                (5, 32, 4, 1500, 4)])
def test_splitkv_multitoken_d128(S, Hq, Hkv, N, splits):
    # up to 32 folded rows per KV head take the wavefront-split decode kernel; (5, 32, 4) has 40 and does not
    c = FC.Case(f"split_mt128_{S}_{Hq}_{Hkv}", B=2, S=S, N=N, Hq=Hq, Hkv=Hkv, D=128, mode="causal", seed=83)
    _say(f"splitkv multi-token d128 S{S} Hq{Hq} Hkv{Hkv} N{N} splits{splits}")
    a = FC.build(c)
    og, lg = run_split(c, a, splits)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where=c.name)


def test_splitkv_workspace_reuse():
    """The workspace needs no initialisation: calls that share one workspace holding arbitrary bytes (different
    splits, shapes and inputs, so a later call's partials overlap an earlier call's differently) must all be
    right."""
    from reax_fmha import ops

    cases = [(FC.Case("reuse_a", B=4, S=1, N=3000, Hq=32, Hkv=8, D=128, mode="causal", seed=90), 16),
             (FC.Case("reuse_b", B=2, S=2, N=777, Hq=16, Hkv=4, D=128, mode="causal", seed=91), 5),
             (FC.Case("reuse_a2", B=4, S=1, N=3000, Hq=32, Hkv=8, D=128, mode="causal", seed=92), 16),
             (FC.Case("reuse_c", B=8, S=1, N=2048, Hq=32, Hkv=8, D=128, mode="causal", seed=93), 16)]
    need = max(ops.splitkv_workspace_bytes(c.B, c.Hkv, c.S * c.G, c.D, n) for c, n in cases)
    gen = torch.Generator(device="cuda").manual_seed(7)
    ws = torch.randint(0, 256, (need,), dtype=torch.uint8, device="cuda", generator=gen)
    for c, n in cases:
        _say(f"splitkv workspace reuse {c.name} splits{n}")
        a = FC.build(c)
        q, k, v = dev(a["q"]), dev(a["k"]), dev(a["v"])
        qpos = torch.from_numpy(a["qpos"]).cuda()
        o, lse = ops.attention_splitkv(q, k, v, qpos, scale=c.scale, num_splits=n, ws=ws)
        torch.cuda.synchronize()
        ref_o, ref_lse = FC.oracle_ref(c, a)
        FC.check_tolerance(host(o), ref_o, lse.cpu().numpy(), ref_lse, where=c.name)


def test_splitkv_graph_replay():
    """A split-KV decode (decode kernel + combine kernel) captured in a HIP graph once and replayed on new
    inputs: every replay equals the eager call on the same inputs bit for bit, with eager calls on the same
    workspace in between."""
    from reax_fmha import ops

    c0 = FC.Case("graph", B=2, S=1, N=1500, Hq=16, Hkv=4, D=128, mode="causal", seed=94)
    n = 8
    a0 = FC.build(c0)
    q, k, v = dev(a0["q"]), dev(a0["k"]), dev(a0["v"])
    qpos = torch.from_numpy(a0["qpos"]).cuda()
    ws = torch.empty(ops.splitkv_workspace_bytes(c0.B, c0.Hkv, c0.G, c0.D, n), dtype=torch.uint8, device="cuda")
    o = torch.empty_like(q)
    lse = torch.empty((c0.B, c0.Hq, 1), dtype=torch.float32, device="cuda")
    run = lambda: ops.attention_splitkv(q, k, v, qpos, scale=c0.scale, num_splits=n, ws=ws, o=o, lse=lse)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for i, seed in enumerate([94, 95, 96, 97]):
        _say(f"splitkv graph replay {i} seed {seed}")
        a = FC.build(FC.Case("graph", B=2, S=1, N=1500, Hq=16, Hkv=4, D=128, mode="causal", seed=seed))
        q.copy_(dev(a["q"]))
        k.copy_(dev(a["k"]))
        v.copy_(dev(a["v"]))
        g.replay()
        torch.cuda.synchronize()
        go, gl = o.clone(), lse.clone()
        eo, el = ops.attention_splitkv(q, k, v, qpos, scale=c0.scale, num_splits=n, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(go, eo) and torch.equal(gl, el), f"replay {i} differs from the eager call"
        if i == 0:
            ref_o, ref_lse = FC.oracle_ref(c0, a)
            FC.check_tolerance(host(go), ref_o, gl.cpu().numpy(), ref_lse, where="graph replay")


def test_splitkv_multitoken_d256():
    c = FC.Case("split_mt", B=2, S=3, N=700, Hq=4, Hkv=2, D=256, mode="causal", seed=82)
    _say("splitkv multi-token d256")
    a = FC.build(c)
    og, lg = run_split(c, a, 5)
    o, lse = FC.oracle_ref(c, a)
    FC.check_tolerance(og, o, lg, lse, where="split_mt")


def test_config4_decode():
    cfg = W.CONFIGS[4]
    _say("config 4 decode split-KV")
    q, k, v, qpos = W.make_decode_inputs(cfg)
    c = FC.Case(cfg.name, B=cfg.B, S=1, N=cfg.N, Hq=cfg.Hq, Hkv=cfg.Hkv, D=cfg.D, mode="qpos", qpos=qpos)
    a = dict(q=q, k=k, v=v, qpos=qpos)
    og, lg = run_split(c, a, cfg.num_splits)
    o, lse = FC.oracle_ref(c, a)
    res = FC.check_tolerance(og, o, lg, lse, where="config4")
    _say(f"  config 4 vs oracle (all rows): {res}")


# ------------------------------------------------------------------------------------------ full-size configs

def test_config2_prefill():
    cfg = W.CONFIGS[2]
    _say("config 2 prefill S4096")
    q, k, v, qpos = W.make_prefill_inputs(cfg)
    c = FC.Case(cfg.name, B=1, S=cfg.S, N=cfg.N, Hq=cfg.Hq, Hkv=cfg.Hkv, D=cfg.D, mode="causal")
    a = dict(q=q, k=k, v=v, qpos=qpos)
    og, lg = run_qx(c, a)
    toks = token_subset(cfg.S, 96, 7)
    o, lse = oracle_on_tokens(c, a, toks)
    res = FC.check_tolerance(og[:, toks], o, lg[:, :, toks], lse, where="config2")
    _say(f"  config 2 vs oracle ({len(toks)} tokens x all heads): {res}")
    res = torch_causal_check(og[0], lg[0], q, k, v, c.G, c.scale, where="config2")
    _say(f"  all {cfg.S} tokens vs float32: {res}")


def test_config5_post():
    cfg = W.CONFIGS[5]
    _say("config 5 long-context gated (reax_fmha_qp) S32768 D256")
    q, k, v, qpos = W.make_prefill_inputs(cfg)
    gate = W.make_gate(cfg)
    c = FC.Case(cfg.name, B=1, S=cfg.S, N=cfg.N, Hq=cfg.Hq, Hkv=cfg.Hkv, D=cfg.D, mode="causal")
    a = dict(q=q, k=k, v=v, qpos=qpos)
    T = cfg.S
    qg = np.empty((T, cfg.Hq, 2 * cfg.D), dtype=np.uint16)
    qg[:, :, : cfg.D] = q[0]
    qg[:, :, cfg.D:] = gate
    del gate
    inv = np.arange(T, dtype=np.int32)
    got = run_post(c, a, qg, inv, T)
    toks = token_subset(cfg.S, 24, 11, edge=16)
    o, _ = oracle_on_tokens(c, a, toks)
    sub_qg = np.ascontiguousarray(qg[toks])
    want = np.zeros((len(toks), cfg.Hq * cfg.D), dtype=np.uint16)
    pyoracle.post_gate(fold_dense(o, c.G), B=1, H=c.Hkv, G=c.G, M=len(toks) * c.G, D=c.D,
                       inv=np.arange(len(toks), dtype=np.int32), Lq=len(toks), qg=sub_qg, qg_rs=cfg.Hq * 2 * cfg.D,
                       out=want, out_rs=cfg.Hq * cfg.D)
    res = FC.check_tolerance(got[toks], W.bf16_bits_to_f32(want).astype(np.float64), where="config5")
    _say(f"  config 5 vs oracle ({len(toks)} tokens x all heads, gated): {res}")
    res = torch_causal_check(got.reshape(T, cfg.Hq, cfg.D), None, q, k, v, c.G, c.scale,
                             gate_bits=qg[:, :, cfg.D:], where="config5")
    _say(f"  all {T} tokens vs float32: {res}")
