"""GPU parity of the drop-in entry points at short query blocks: reax_fmha_q (both libraries) and reax_fmha_qp with at
most 64 folded rows per (batch, KV head), the engine's decode shape (Lq 1 x G 8 = 8 rows; reax_fmha_v8.cu:141-162,
224-235; reax_fmha_v11.cu:451-522, 583-590). Every result is checked against the double-precision oracle in drop-in
mode (the reference's block-wide qpos = 0 rule), to the bar of the path: bf16 outputs max-abs <= 2e-2 and
mean-abs <= 2e-3; rows of a 64-row block whose largest qpos is 0 must be V[0] bit for bit, rows with qpos < 0
outside such a block exactly 0, and POST rows not named by inv untouched."""
import numpy as np
import pytest

import fmha_cases as FC
import pyoracle
from reax_fmha import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _say(msg):
    print(f"[gpu-dropin-short] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from reax_fmha import abi

    abi.howu()
    abi.post()


def dev(bits):
    return W.bits_to_torch(bits, "cuda")


def fold(x, G):
    """natural [B][S][Hq][D] -> folded [B][Hkv][S*G][D] (row r = token r/G, query head h*G + r%G)."""
    B, S, Hq, D = x.shape
    return np.ascontiguousarray(x.reshape(B, S, Hq // G, G, D).transpose(0, 2, 1, 3, 4).reshape(B, Hq // G, S * G, D))


def unfold(x, G):
    B, H, M, D = x.shape
    return x.reshape(B, H, M // G, G, D).transpose(0, 2, 1, 3, 4).reshape(B, M // G, H * G, D)


def decode_qpos(B, S, N, lens=None):
    """qpos [B][S] of S new tokens appended to caches of `lens` keys (default N): token m sees keys 0..len-S+m."""
    lens = [N] * B if lens is None else lens
    return np.stack([np.arange(S, dtype=np.int32) + (L - S) for L in lens]).astype(np.int32)


def run_q(c, a, lib):
    from reax_fmha import ops

    q = dev(fold(a["q"], c.G))
    k, v = dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(np.ascontiguousarray(a["qpos"])).cuda()
    o = torch.full_like(q, float("nan"))
    ops.fmha_q(q, k, v, qpos, c.G, o, c.scale, lib=lib)
    torch.cuda.synchronize()
    return unfold(W.torch_to_bits(o), c.G)


def run_qp(c, a, qg_bits, inv, T):
    from reax_fmha import ops

    q = dev(fold(a["q"], c.G))
    k, v = dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(np.ascontiguousarray(a["qpos"])).cuda()
    out = torch.from_numpy(np.full((T, c.Hq * c.D), 0x7E00, dtype=np.uint16).view(np.int16)).cuda().view(torch.bfloat16)
    ops.fmha_qp(q, k, v, qpos, c.G, c.scale, torch.from_numpy(inv).cuda(), c.S, dev(qg_bits), out)
    torch.cuda.synchronize()
    return W.torch_to_bits(out)


def v0_rows(c, a):
    """(batch, token, query head) of every row the drop-in rule stores as V[0]: rows of a 64-row block of (b, h)
    whose largest raw qpos is 0."""
    out = []
    M = c.S * c.G
    for b in range(c.B):
        qp = a["qpos"][b]
        for j in range(0, M, 64):
            rows = range(j, min(j + 64, M))
            if max(int(qp[r // c.G]) for r in rows) == 0:
                for h in range(c.Hkv):
                    out += [(b, r // c.G, h * c.G + r % c.G) for r in rows]
    return out


def check_rules(c, a, og):
    """V[0] bit for bit on the block-rule rows, exact zeros on the other qpos < 0 rows."""
    v0 = v0_rows(c, a)
    s0 = set(v0)
    for b, m, hq in v0:
        assert (og[b, m, hq] == a["v"][b, 0, hq // c.G]).all(), f"b{b} token {m} head {hq}: V[0] expected"
    for b in range(c.B):
        for m in range(c.S):
            if a["qpos"][b, m] < 0:
                for hq in range(c.Hq):
                    if (b, m, hq) not in s0:
                        assert (og[b, m, hq] == 0).all(), f"b{b} token {m} head {hq}: 0 expected"
    return len(v0)


# (B, S, G, Hkv, N, cache lengths): M = S*G folded rows per (b, KV head), all <= 64. N is never a multiple of the
# 64-key tile, so the last key tile is partial; the cache lengths differ per batch entry.
SHORT = [
    (3, 1, 8, 2, 1000, [1000, 513, 1]),  # the engine's decode step: Lq 1 x G 8 = 8 rows
    (2, 5, 8, 1, 777, [777, 64]),        # M = 40
    (2, 8, 8, 2, 300, [300, 9]),         # M = 64: one full block
    (1, 16, 4, 1, 129, None),            # M = 64 at G = 4
    (2, 3, 16, 2, 5003, [5003, 4100]),   # M = 48, a long cache
]


@pytest.mark.parametrize("lib", ["howu", "post"])
@pytest.mark.parametrize("shape", SHORT, ids=lambda s: f"B{s[0]}_S{s[1]}_G{s[2]}_H{s[3]}_N{s[4]}")
def test_reax_fmha_q_short(lib, shape):
    B, S, G, Hkv, N, lens = shape
    qp = decode_qpos(B, S, N, lens)
    c = FC.Case(f"q_short_{lib}", B=B, S=S, N=N, Hq=G * Hkv, Hkv=Hkv, D=256, mode="qpos", seed=500 + S * G + N % 997,
                qpos=qp)
    _say(f"reax_fmha_q {lib} B{B} S{S} G{G} Hkv{Hkv} N{N} (M = {S * G})")
    a = FC.build(c)
    og = run_q(c, a, lib)
    oref, _ = FC.oracle_ref(c, a, dropin=True)
    res = FC.check_tolerance(og, oref, where=c.name)
    check_rules(c, a, og)
    _say(f"  {res}")


def _rule_cases():
    """Block-rule patterns inside one short block: G = 8, S = 8 (one 64-row block) with qpos {0, -1 x 7} (the
    whole block is V[0]) and {5, -1, 0, -1, 2, -1, -1, 0} (per-row rules); S = 1 decode steps whose cache holds one
    key ({0}: V[0]), none ({-1}: 0) or all of them."""
    N = 70
    return [
        FC.Case("blk_0_neg7", B=1, S=8, N=N, Hq=16, Hkv=2, D=256, mode="qpos", seed=531,
                qpos=np.array([[0, -1, -1, -1, -1, -1, -1, -1]], dtype=np.int32)),
        FC.Case("blk_mixed", B=1, S=8, N=N, Hq=16, Hkv=2, D=256, mode="qpos", seed=532,
                qpos=np.array([[5, -1, 0, -1, 2, -1, -1, 0]], dtype=np.int32)),
        FC.Case("decode_first_token", B=3, S=1, N=N, Hq=16, Hkv=2, D=256, mode="qpos", seed=533,
                qpos=np.array([[0], [-1], [N - 1]], dtype=np.int32)),
    ]


@pytest.mark.parametrize("lib", ["howu", "post"])
@pytest.mark.parametrize("ci", [0, 1, 2], ids=["blk_0_neg7", "blk_mixed", "decode_first_token"])
def test_reax_fmha_q_short_block_rule(lib, ci):
    c = _rule_cases()[ci]
    _say(f"reax_fmha_q block rule {lib} {c.name}")
    a = FC.build(c)
    og = run_q(c, a, lib)
    oref, _ = FC.oracle_ref(c, a, dropin=True)
    FC.check_tolerance(og, oref, where=c.name)
    n = check_rules(c, a, og)
    if ci != 1:
        assert n > 0, "the case must hold a block whose largest qpos is 0"


def _post_case(c, a, seed, drop=()):
    """inv [B][Lq]: a permutation of T = B*S + 3 output rows, with the (batch, token) pairs in `drop` set to -1."""
    rng = np.random.default_rng(seed)
    T = c.B * c.S + 3
    inv = rng.permutation(T)[: c.B * c.S].astype(np.int32).reshape(c.B, c.S)
    for b, m in drop:
        inv[b, m] = -1
    qg = W.bf16_normal(rng, (T, c.Hq, 2 * c.D))
    return inv, qg, T


@pytest.mark.parametrize("ci", [0, 1, 2, 3])
def test_reax_fmha_qp_short(ci):
    """The POST epilogue at short query blocks: decode steps (M = 8, one with a one-key cache: the block rule),
    M = 40 and M = 64 with padding rows (inv < 0), checked bit for bit where the oracle's output is exact and to the
    tolerance elsewhere; rows not named by inv keep their sentinel."""
    N = 1000
    cases = [
        (FC.Case("qp_decode", B=3, S=1, N=N, Hq=16, Hkv=2, D=256, mode="qpos", seed=541,
                 qpos=decode_qpos(3, 1, N, [1000, 1, 400])), [(2, 0)]),
        (FC.Case("qp_decode_first", B=2, S=1, N=N, Hq=16, Hkv=2, D=256, mode="qpos", seed=542,
                 qpos=np.array([[0], [999]], dtype=np.int32)), []),
        (FC.Case("qp_m40", B=2, S=5, N=N, Hq=8, Hkv=1, D=256, mode="qpos", seed=543,
                 qpos=decode_qpos(2, 5, N, [1000, 300])), [(0, 1), (1, 4)]),
        (FC.Case("qp_m64", B=1, S=8, N=N, Hq=16, Hkv=2, D=256, mode="qpos", seed=544,
                 qpos=np.array([[5, -1, 0, -1, 2, 999, 998, 0]], dtype=np.int32)), [(0, 3)]),
    ]
    c, drop = cases[ci]
    _say(f"reax_fmha_qp short {c.name} B{c.B} S{c.S} G{c.G} (M = {c.S * c.G})")
    a = FC.build(c)
    inv, qg, T = _post_case(c, a, 550 + ci, drop)
    got = run_qp(c, a, qg, inv, T)
    o, _ = FC.oracle_ref(c, a, dropin=True)
    want = np.full((T, c.Hq * c.D), 0x7E00, dtype=np.uint16)
    of = o.reshape(c.B, c.S, c.Hkv, c.G, c.D).transpose(0, 2, 1, 3, 4).reshape(c.B, c.Hkv, c.S * c.G, c.D)
    pyoracle.post_gate(of, B=c.B, H=c.Hkv, G=c.G, M=c.S * c.G, D=c.D, inv=inv, Lq=c.S, qg=qg,
                       qg_rs=c.Hq * 2 * c.D, out=want, out_rs=c.Hq * c.D)
    untouched = np.setdiff1d(np.arange(T), inv[inv >= 0])
    assert (got[untouched] == 0x7E00).all(), "rows not named by inv must stay untouched"
    rows = inv[inv >= 0]
    FC.check_tolerance(got[rows], W.bf16_bits_to_f32(want[rows]).astype(np.float64), where=c.name)
    # rows whose attention output is exactly V[0] (block rule) or 0 (qpos < 0): the gated result is exact too
    exact = set(v0_rows(c, a))
    for b in range(c.B):
        for m in range(c.S):
            if a["qpos"][b, m] < 0:
                exact |= {(b, m, hq) for hq in range(c.Hq)}
    for b, m, hq in exact:
        R = inv[b, m]
        if R >= 0:
            sl = slice(hq * c.D, (hq + 1) * c.D)
            assert (got[R, sl] == want[R, sl]).all(), f"{c.name}: b{b} token {m} head {hq} not bit-exact"


def test_varlen_d256_short():
    """reax_fmha_varlen at head_dim 256 with max_seqlen * G <= 64 (every sequence one short row block)."""
    from reax_fmha import ops

    c = FC.Case("varlen_d256_short", B=1, S=0, N=0, Hq=16, Hkv=2, D=256, mode="varlen", seed=561,
                seqlens=[5, 8, 0, 3, 1, 7])
    _say(f"varlen d256 short {c.seqlens} G{c.G}")
    a = FC.build(c)
    q, k, v = dev(a["q"]), dev(a["k"]), dev(a["v"])
    cu = torch.from_numpy(a["cu"]).cuda()
    o, lse = ops.attention_varlen(q, k, v, cu, max(c.seqlens), scale=c.scale)
    torch.cuda.synchronize()
    ref_o, ref_lse = FC.oracle_ref(c, a)
    FC.check_tolerance(W.torch_to_bits(o), ref_o, lse.cpu().numpy(), ref_lse, where=c.name)


# ---------------------------------------------------------------------------------------- split-KV behind the ABI
# At most 32 folded rows and long enough key ranges, reax_fmha_q / reax_fmha_qp split the keys across the GPU
# (fmha_short.hip: the decode kernel per split, partials in the library's static scratch, an LSE combine that
# applies the entry point's store). These shapes take that path; the cache lengths differ per batch entry, so
# some splits see no key at all, and one entry's cache holds one key (the block rule: V[0]).

SPLIT = [
    (1, 1, 8, 2, 32768, None),                     # the bench's batch-1 decode step
    (2, 4, 8, 1, 9000, [9000, 4500]),              # M = 32: four tokens of 8 heads
    (4, 1, 16, 2, 3000, [3000, 1, 2999, 64]),      # G = 16
    (3, 3, 8, 2, 20000, [20000, 2, 7777]),         # M = 24, a two-key cache
]


@pytest.mark.parametrize("lib", ["howu", "post"])
@pytest.mark.parametrize("shape", SPLIT, ids=lambda s: f"B{s[0]}_S{s[1]}_G{s[2]}_H{s[3]}_N{s[4]}")
def test_reax_fmha_q_split(lib, shape):
    test_reax_fmha_q_short(lib, shape)


@pytest.mark.parametrize("qmode", ["decode", "beyond"])
def test_reax_fmha_qp_split(qmode):
    """reax_fmha_qp on the split path, B 5 decode steps over a 12000-key cache: per-entry cache lengths ('decode'),
    or qpos past the cache's end for some entries (they see every key) and -1 for one (nothing: O = 0)."""
    N, B = 12000, 5
    qp = decode_qpos(B, 1, N, [12000, 1, 6000, 130, 11999]) if qmode == "decode" else \
        np.array([[N + 5], [-1], [N - 1], [2 * N], [0]], dtype=np.int32)
    c = FC.Case(f"qp_split_{qmode}", B=B, S=1, N=N, Hq=16, Hkv=2, D=256, mode="qpos", seed=571, qpos=qp)
    _say(f"reax_fmha_qp split {qmode} B{B} N{N}")
    a = FC.build(c)
    inv, qg, T = _post_case(c, a, 572, drop=[(3, 0)])
    got = run_qp(c, a, qg, inv, T)
    o, _ = FC.oracle_ref(c, a, dropin=True)
    want = np.full((T, c.Hq * c.D), 0x7E00, dtype=np.uint16)
    of = o.reshape(c.B, c.S, c.Hkv, c.G, c.D).transpose(0, 2, 1, 3, 4).reshape(c.B, c.Hkv, c.S * c.G, c.D)
    pyoracle.post_gate(of, B=c.B, H=c.Hkv, G=c.G, M=c.S * c.G, D=c.D, inv=inv, Lq=c.S, qg=qg,
                       qg_rs=c.Hq * 2 * c.D, out=want, out_rs=c.Hq * c.D)
    untouched = np.setdiff1d(np.arange(T), inv[inv >= 0])
    assert (got[untouched] == 0x7E00).all(), "rows not named by inv must stay untouched"
    rows = inv[inv >= 0]
    FC.check_tolerance(got[rows], W.bf16_bits_to_f32(want[rows]).astype(np.float64), where=c.name)
    for b in range(B):
        R = inv[b, 0]
        if R >= 0 and (a["qpos"][b, 0] <= 0):  # V[0] (block rule) or 0: exact
            assert (got[R] == want[R]).all(), f"{c.name}: entry {b} not bit-exact"


def test_short_split_two_streams():
    """Calls on two streams share the library's split scratch: each stream's calls are queued without host
    synchronisation, alternating, into separate outputs; every output must equal the same call made alone on the
    default stream, bit for bit (the split path is deterministic)."""
    from reax_fmha import ops

    N, B, G, Hkv = 6000, 3, 8, 2
    cases = []
    for i in range(6):
        c = FC.Case(f"streams_{i}", B=B, S=1, N=N, Hq=G * Hkv, Hkv=Hkv, D=256, mode="qpos", seed=580 + i,
                    qpos=decode_qpos(B, 1, N, [N - 7 * i, N // (i + 1), 100 * i + 1]))
        a = FC.build(c)
        q = dev(fold(a["q"], G))
        cases.append((c, q, dev(a["k"]), dev(a["v"]), torch.from_numpy(a["qpos"]).cuda()))
    _say("split scratch shared by two streams")
    alone = []
    for c, q, k, v, qpos in cases:
        o = torch.empty_like(q)
        ops.fmha_q(q, k, v, qpos, G, o, c.scale, lib="post")
        alone.append(o)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for i, (c, q, k, v, qpos) in enumerate(cases):
        with torch.cuda.stream(s1 if i % 2 == 0 else s2):
            o = torch.full_like(q, float("nan"))
            ops.fmha_q(q, k, v, qpos, G, o, c.scale, lib="post")
            outs.append(o)
    torch.cuda.synchronize()
    for i, (o, ref) in enumerate(zip(outs, alone)):
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16)), f"call {i} differs from the same call alone"
    c, q, k, v, qpos = cases[0]
    a = FC.build(c)
    oref, _ = FC.oracle_ref(c, a, dropin=True)
    FC.check_tolerance(unfold(W.torch_to_bits(outs[0]), G), oref, where="two streams")


def test_short_split_graph_capture():
    """Under graph capture the drop-in entry point runs unsplit (the capture must not depend on the split scratch
    or its events); the captured call replays correctly on new inputs, and eager calls between the replays still
    take the split path."""
    from reax_fmha import ops

    N, B, G, Hkv = 5000, 2, 8, 2
    c = FC.Case("graph_short", B=B, S=1, N=N, Hq=G * Hkv, Hkv=Hkv, D=256, mode="qpos", seed=590,
                qpos=decode_qpos(B, 1, N, [N, 3000]))
    a = FC.build(c)
    q, k, v = dev(fold(a["q"], G)), dev(a["k"]), dev(a["v"])
    qpos = torch.from_numpy(a["qpos"]).cuda()
    o = torch.empty_like(q)
    run = lambda: ops.fmha_q(q, k, v, qpos, G, o, c.scale, lib="howu")
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
    for i, seed in enumerate([591, 592, 593]):
        _say(f"graph replay {i} seed {seed}")
        ci = FC.Case("graph_short", B=B, S=1, N=N, Hq=G * Hkv, Hkv=Hkv, D=256, mode="qpos", seed=seed,
                     qpos=c.qpos)
        ai = FC.build(ci)
        q.copy_(dev(fold(ai["q"], G)))
        k.copy_(dev(ai["k"]))
        v.copy_(dev(ai["v"]))
        g.replay()
        torch.cuda.synchronize()
        got = unfold(W.torch_to_bits(o), G)
        eager = torch.empty_like(q)
        ops.fmha_q(q, k, v, qpos, G, eager, c.scale, lib="howu")
        torch.cuda.synchronize()
        oref, _ = FC.oracle_ref(ci, ai, dropin=True)
        FC.check_tolerance(got, oref, where=f"replay {i}")
        FC.check_tolerance(unfold(W.torch_to_bits(eager), G), oref, where=f"eager {i}")
