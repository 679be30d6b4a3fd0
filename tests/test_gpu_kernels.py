"""Kernel-level parity of the HIP path against the CPU oracle (through the C ABI).

Integer/index work (top-k, tree layout, sampling, acceptance, KV gather) must
be bit-exact; floating-point contractions are checked with the tolerance the
north star states: max|a-b|/max|b| <= 2e-2 in bf16 and <= 1e-5 in fp32.
"""
import numpy as np
import pytest
import torch

from oracle import kv as OK
from oracle import sampling as OS
from oracle import tree as OT
from oracle import model as OM

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from flashgrpo_amd import _lib

    _lib.load()


def K():
    from flashgrpo_amd import kernels

    return kernels


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def to_np(t):
    return t.detach().float().cpu().numpy()


def noise_i32(n_rows, n_cols, seed):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 2 ** 32, size=(n_rows, n_cols), dtype=np.uint64)
    return u, torch.from_numpy(u.astype(np.uint32).view(np.int32)).to(DEV)


# ------------------------------------------------------------------ KV gather
@pytest.mark.parametrize("dtype,width", [(torch.bfloat16, 5), (torch.float32, 5), (torch.bfloat16, 12)])
def test_kv_path_gather_matches_oracle(dtype, width):
    """Paths with self-copies, crossing rows (a destination that is an earlier row's
    source, and a swap) and, at width 12, the long-path kernel."""
    torch.manual_seed(0)
    L, B, H, S, D = 3, 5, 2, 40, 128 if dtype == torch.bfloat16 else 64
    caches = [torch.randn(B, H, S, D, device=DEV).to(dtype) for _ in range(2 * L)]
    before = [to_np(c) for c in caches]
    seq = np.array([3, 10, 0, 20, 7], np.int32)
    paths = [[0, 2, 5, 7], [0], [0, 2, 1], [0, 3, 4], [0, 6, 8, 9, 11]]
    if width > 8:
        paths[3] = [0, 2, 5, 7, 9, 10, 13, 14, 15, 16, 17, 19]
    nodes = np.zeros((B, width), np.int32)
    for b, p in enumerate(paths):
        nodes[b, :len(p)] = p
    lens = np.array([len(p) for p in paths], np.int32)
    ptrs = torch.tensor([c.data_ptr() for c in caches], dtype=torch.int64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    c0 = caches[0]
    K().kv_path_gather(ptrs, batch=B, kv_heads=H, head_dim=D, elem_bytes=c0.element_size(),
                       strides=(c0.stride(0), c0.stride(1), c0.stride(2)), capacity=S,
                       seq_len=torch.from_numpy(seq).to(DEV), acc_nodes=torch.from_numpy(nodes).to(DEV),
                       acc_len=torch.from_numpy(lens).to(DEV), tree_nodes=20, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    for c, bef in zip(caches, before):
        want = OK.compact_rows(bef, seq, nodes, lens)
        assert np.array_equal(to_np(c), want)


def test_kv_path_gather_seed17_golden_and_bounds():
    import json
    import os

    gold = os.path.join(os.path.dirname(__file__), "golden")
    arr = np.load(os.path.join(gold, "reference_arrays.npz"))
    case = json.load(open(os.path.join(gold, "reference_cases.json")))["seed17_kv"]
    # head_dim 8 fp32 rows are 32 bytes: multiple of 16, so the kernel accepts them
    key = torch.from_numpy(arr["seed17_key"]).to(DEV).contiguous()
    val = torch.from_numpy(arr["seed17_value"]).to(DEV).contiguous()
    B, H, S, D = key.shape
    acc = case["accepted"]
    nodes = torch.tensor([p + [p[-1]] * (3 - len(p)) for p in acc], dtype=torch.int32, device=DEV)
    lens = torch.tensor([len(p) for p in acc], dtype=torch.int32, device=DEV)
    seq = torch.full((B,), case["old_len"], dtype=torch.int32, device=DEV)
    ptrs = torch.tensor([key.data_ptr(), val.data_ptr()], dtype=torch.int64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    K().kv_path_gather(ptrs, batch=B, kv_heads=H, head_dim=D, elem_bytes=4, strides=(key.stride(0), key.stride(1), D),
                       capacity=S, seq_len=seq, acc_nodes=nodes, acc_len=lens, tree_nodes=4, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    old = case["old_len"]
    for b, p in enumerate(acc):
        n = len(p)
        assert np.array_equal(to_np(key)[b, :, :old + n], arr["seed17_expect_key"][b, :, :old + n])
        assert np.array_equal(to_np(val)[b, :, :old + n], arr["seed17_expect_value"][b, :, :old + n])
    # out-of-range node: flagged, row untouched
    before = to_np(key).copy()
    bad = torch.tensor([[0, 4, 4], [0, 1, 1]], dtype=torch.int32, device=DEV)
    K().kv_path_gather(ptrs, batch=B, kv_heads=H, head_dim=D, elem_bytes=4, strides=(key.stride(0), key.stride(1), D),
                       capacity=S, seq_len=seq, acc_nodes=bad, acc_len=torch.tensor([2, 2], dtype=torch.int32,
                                                                                    device=DEV),
                       tree_nodes=4, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    assert np.array_equal(to_np(key)[0], before[0])
    # a path longer than the tree (3 accepted rows, 2 tree nodes): flagged, rows untouched
    err.zero_()
    before = to_np(key).copy()
    K().kv_path_gather(ptrs, batch=B, kv_heads=H, head_dim=D, elem_bytes=4, strides=(key.stride(0), key.stride(1), D),
                       capacity=S, seq_len=seq, acc_nodes=torch.tensor([[0, 1, 1], [0, 1, 1]], dtype=torch.int32,
                                                                       device=DEV),
                       acc_len=torch.tensor([3, 1], dtype=torch.int32, device=DEV), tree_nodes=2, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    assert np.array_equal(to_np(key), before)


# ------------------------------------------------------------------ top-k / layout
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("V,kmax", [(37, 3), (1000, 4), (32000, 8), (152064, 4), (5000, 16), (9, 1)])
def test_medusa_topk_matches_canonical_order(dtype, V, kmax):
    g = torch.Generator(device="cpu").manual_seed(V + kmax)
    R = 24
    x = torch.randn(R, V, generator=g)
    x[:4] = torch.round(x[:4] * 2) / 2          # heavy ties
    x[4, :] = 0.0
    x[5, ::3] = -0.0
    xd = x.to(dtype).to(DEV)
    tok, sc, st = K().medusa_topk(xd, kmax, stats=True)
    xs = to_np(xd)
    for r in range(R):
        ids, vals = OT.topk_canonical(xs[r], kmax)
        assert tok[r].tolist() == ids.tolist(), r
        assert np.array_equal(to_np(sc[r]), vals.astype(np.float32) + 0.0)
        lse = np.log(np.sum(np.exp(xs[r].astype(np.float64) - xs[r].max()))) + xs[r].max()
        assert abs(float(st[r, 1]) - lse) < 1e-4 * max(1.0, abs(lse))
        assert float(st[r, 0]) == float(xs[r].max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_medusa_topk_sanitize_nan_inf(dtype):
    """sanitize=1 ranks nan_to_num(x, -1e9, 1e9, -1e9) (chain builder); sanitize=0 ranks
    NaN above every number (torch.topk)."""
    g = torch.Generator(device="cpu").manual_seed(12)
    R, V, k = 6, 4099, 4
    x = torch.randn(R, V, generator=g)
    x[0, [5, 77, 4000]] = float("nan")
    x[1, [3, 9]] = float("inf")
    x[2, :] = float("-inf")
    x[3, :] = float("nan")
    x[4, ::2] = float("-inf")
    x[5, [10, 11]] = float("nan")
    x[5, [12]] = float("inf")
    xd = x.to(dtype).to(DEV)
    xs = to_np(xd)
    tok, sc, st = K().medusa_topk(xd, k, stats=True, sanitize=True)
    raw, _, _ = K().medusa_topk(xd, k)
    for r in range(R):
        clean = OT.nan_to_num_logits(xs[r])
        ids, vals = OT.topk_canonical(clean, k)
        assert tok[r].tolist() == ids.tolist(), r
        assert np.array_equal(to_np(sc[r]), vals.astype(np.float32) + 0.0), r
        m = float(clean.max())
        lse = np.log(np.sum(np.exp(clean.astype(np.float64) - m))) + m
        assert float(st[r, 0]) == m and abs(float(st[r, 1]) - lse) < 1e-4 * max(1.0, abs(lse)), r
        assert raw[r].tolist() == OT.topk_canonical(xs[r], k)[0].tolist(), r


def test_tree_layout_matches_oracle_trees():
    rng = np.random.default_rng(3)
    for ks, budget, B, V in [([4, 2], 16, 8, 500), ([4, 2, 1, 1], 32, 6, 300), ([4, 3, 2], 16, 3, 64)]:
        logits = [rng.standard_normal((B, V)).astype(np.float32) for _ in ks]
        roots = rng.integers(0, V, B)
        plan = OT.Plan(budget, len(ks), ks, OT.dense_node_count(ks), "fixed", "dense")
        trees = OT.build_batch_trees(roots, logits, plan)
        parents, depths, ranks = OT.dense_topology(ks, budget)
        N = len(parents)
        lg = torch.from_numpy(np.concatenate(logits)).to(DEV)
        tok, sc, _ = K().medusa_topk(lg, max(ks))
        out, scores = K().tree_layout(tok, sc, B, torch.from_numpy(roots.astype(np.int32)).to(DEV),
                                      torch.tensor(depths, dtype=torch.int32, device=DEV),
                                      torch.tensor(ranks, dtype=torch.int32, device=DEV), N)
        for b, t in enumerate(trees):
            assert out[b].tolist() == t.tokens
            assert np.allclose(to_np(scores[b]), np.array(t.scores, np.float32))


SPARSE_CASES = [  # nodes_by_head, budget, vocab, temperature, penalty, gate
    ([4, 3, 2], 10, 17, 1.0, 0.05, None),
    ([4, 3, 2], 32, 300, 0.7, 0.05, "random"),
    ([5, 4], 16, 500, 1.0, 0.0, None),
    ([3, 4, 3], 14, 64, 1.0, 0.3, "random"),
    ([6, 0, 3], 12, 40, 1.3, 0.05, None),
    ([2, 2, 2, 2], 9, 50, 1.0, 0.05, "random"),
    ([4, 3, 2], 8, 5, 1.0, 0.05, None),
    ([3], 8, 100, 1.0, 0.05, None),
    ([8, 8, 8], 40, 1000, 0.5, 0.01, "random"),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", range(len(SPARSE_CASES)))
def test_sparse_tree_layout_matches_oracle(dtype, case):
    """fg_sparse_tree_layout (flashgrpo_b200/decoding/medusa_tree.py:509-685) against the
    oracle's greedy builder: tokens, parents, depths, node counts and fp64 path scores
    bit-exact, including ties, NaN rows, a per-row head-3 gate and vocabularies
    narrower than the head widths."""
    from flashgrpo_amd.decoding.medusa_tree import TreePlan, sparse_max_nodes, sparse_tree_device, sparse_widths

    nodes, budget, V, temp, pen, gate = SPARSE_CASES[case]
    B = 11
    rng = np.random.default_rng(100 + case)
    heads = min(len(nodes), 3)
    x = rng.standard_normal((heads * B, V)).astype(np.float32)
    x[:3] = np.round(x[:3] * 2) / 2          # ties inside a row and across parents
    if heads >= 2:
        x[B + 1, : V // 2] = np.nan          # a head-2 row with NaN candidates
    x[4] = 0.0                               # an all-equal row
    xd = torch.from_numpy(x).to(dtype).to(DEV)
    xs = to_np(xd).astype(np.float32)
    roots = rng.integers(0, V, B)
    g = rng.random(B) < 0.5 if gate == "random" else None
    plan = TreePlan(budget, len(nodes), list(nodes), 1 + sum(nodes), "fixed", "sparse_asymmetric", list(nodes), 1, 8,
                    temp, pen)
    oplan = OT.Plan(budget, len(nodes), list(nodes), 1 + sum(nodes), "fixed", "sparse_asymmetric", list(nodes), 1, 8,
                    temp, pen)
    want = OT.build_sparse_trees(roots, [xs[h * B:(h + 1) * B] for h in range(heads)], oplan,
                                 None if g is None else g.tolist())
    kc = max(sparse_widths(nodes[:3], V))
    tok, sc, _ = K().medusa_topk(xd, kc)
    gd = None if g is None else torch.from_numpy(g).to(DEV)
    d = sparse_tree_device(torch.from_numpy(roots.astype(np.int32)).to(DEV), tok, sc, plan, B, V, head3_gate=gd,
                           scores=True)
    N = sparse_max_nodes(plan)
    assert d["tokens"].shape == (B, N)
    got = {k: v.cpu().numpy() for k, v in d.items()}
    for b, t in enumerate(want):
        n = t.node_count
        assert n <= N
        assert int(got["n_nodes"][b]) == n, b
        assert got["tokens"][b, :n].tolist() == t.tokens, b
        assert got["parents"][b, :n].tolist() == t.parents, b
        assert got["depth"][b, :n].tolist() == t.depths, b
        assert got["scores"][b, :n].tolist() == t.scores, b
        assert got["pos_offset"][b, :n].tolist() == [x - 1 for x in t.depths]
        bits = OT.ancestor_bits(t.parents)
        assert [int(v) & 0xFFFFFFFFFFFFFFFF for v in got["anc"][b, :n]] == bits, b
        assert got["n_children"][b, :n].tolist() == [len(t.children(i)) for i in range(n)]
        # padding: self-only mask, never a child, offset 0
        assert got["parents"][b, n:].tolist() == [-1] * (N - n)
        assert [int(v) & 0xFFFFFFFFFFFFFFFF for v in got["anc"][b, n:]] == [1 << i for i in range(n, N)]
        assert not got["pos_offset"][b, n:].any()


# ------------------------------------------------------------------ sampling
MODES = [dict(), dict(temperature=0.7), dict(temperature=1.3, top_p=0.95), dict(top_p=0.5), dict(top_k=5),
         dict(top_k=50, top_p=0.8, temperature=0.9), dict(greedy=True), dict(temperature=0.0),
         dict(temperature=None), dict(top_p=0.999)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mode", MODES, ids=[str(m) for m in MODES])
def test_sample_tokens_bit_exact(dtype, mode):
    g = torch.Generator(device="cpu").manual_seed(11)
    rows = []
    for V, scale in [(4, 1.0), (37, 3.0), (1000, 2.0), (32000, 1.0), (32000, 6.0)]:
        for r in range(6):
            x = torch.randn(V, generator=g) * scale
            if r == 0:
                x = torch.zeros(V)
            if r == 1:
                x = torch.round(x)
            rows.append(x)
    for x in rows:
        V = x.numel()
        xd = x.to(dtype).to(DEV).reshape(1, V).repeat(8, 1)
        u, nz = noise_i32(8, 1, V)
        out = K().sample_tokens(xd, noise=nz, temperature=mode.get("temperature", 1.0),
                                greedy=mode.get("greedy", False), top_k=mode.get("top_k"),
                                top_p=mode.get("top_p", 1.0))
        xs = to_np(xd[0])
        want = [OS.sample_row(xs, int(u[i, 0]), do_sample=not mode.get("greedy", False),
                              temperature=mode.get("temperature", 1.0), top_p=mode.get("top_p", 1.0),
                              top_k=mode.get("top_k")) for i in range(8)]
        assert out.tolist() == want, (V, mode)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mode", [{}, {"temperature": 0.7}, {"greedy": True}, {"temperature": 1.3}])
def test_split_sampling_equals_single_workgroup(dtype, mode):
    """Rows split over 16 workgroups (unrestricted / greedy draws: chunk maxima, then one
    draw launch) give the tokens of the one-workgroup-per-row kernel, including flat rows,
    ties, -inf and NaN entries, rows of only -inf or NaN, and short vocabularies. The
    vocabularies put the chunk end (V / 16 rounded up to 8) inside the first load group,
    inside the last group of a pass, exactly at a pass end and one step into a second pass
    (the 1.5B, 8B and 7B vocabularies among them)."""
    g = torch.Generator(device="cpu").manual_seed(23)
    for V in (5, 37, 1000, 32000, 128256, 131072, 131200, 151936, 152064):
        x = torch.randn(48, V, generator=g) * 2.0
        x[0] = 0.0
        x[1] = torch.round(x[1])
        x[2, V // 3] = 30.0
        x[3, : V // 2] = float("-inf")
        x[4, V - 1] = float("nan")
        x[5] = float("-inf")
        x[6] = float("nan")
        xd = x.to(dtype).to(DEV)
        for draw in range(3):
            kw = dict(seed=99, step=draw, draw=draw, temperature=mode.get("temperature", 1.0),
                      greedy=mode.get("greedy", False))
            a = K().sample_tokens(xd, split=True, **kw)
            b = K().sample_tokens(xd, split=False, **kw)
            assert a.tolist() == b.tolist(), (V, mode, draw)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mode", [{"top_p": 0.95}, {"top_p": 0.5, "temperature": 0.7}, {"top_p": 0.999},
                                  {"top_p": 0.9, "temperature": 1.3}])
def test_split_top_p_equals_single_workgroup(dtype, mode):
    """Top-p draws split over 16 workgroups (seven launches: max, four radix levels,
    cut, pick) give the tokens of the one-workgroup radix select, on flat rows, heavy
    ties, a dominant token, -inf / NaN entries and vocabularies shorter than the
    chunk count; a few rows are also checked against the oracle."""
    g = torch.Generator(device="cpu").manual_seed(31)
    for V in (5, 37, 1000, 32000, 152064):
        x = torch.randn(40, V, generator=g) * 2.0
        x[0] = 0.0
        x[1] = torch.round(x[1])
        x[2, V // 3] = 30.0
        x[3, : V // 2] = float("-inf")
        x[4] = torch.round(x[4] * 4) / 4
        if V > 8:
            x[5, 3] = float("nan")
        xd = x.to(dtype).to(DEV)
        for draw in range(2):
            kw = dict(seed=77, step=draw, draw=draw, temperature=mode.get("temperature", 1.0), top_p=mode["top_p"])
            a = K().sample_tokens(xd, split=True, **kw)
            b = K().sample_tokens(xd, split=False, **kw)
            assert a.tolist() == b.tolist(), (V, mode, draw)
        xs = to_np(xd)
        for i in (0, 1, 2, 4, 7):
            want = OS.sample_row(xs[i], OS.counter_noise(77, 1, i, 1), temperature=mode.get("temperature", 1.0),
                                 top_p=mode["top_p"])
            assert int(a[i]) == want, (V, mode, i)


def test_split_top_p_walk_step_equals_single_workgroup():
    """The lazy walk's top-p draws (active rows only) through the split path equal the
    one-workgroup walk step, step by step."""
    rng = np.random.default_rng(12)
    B, ks, budget, V = 16, [4, 2, 1], 16, 3000
    trees, parents, N, slots, packed = _walk_case(rng, B, ks, budget, V, True)
    tt = torch.tensor([t.tokens for t in trees], dtype=torch.int32, device=DEV)
    pp = torch.tensor([parents] * B, dtype=torch.int32, device=DEV)
    nn = torch.full((B,), N, dtype=torch.int32, device=DEV)
    D = len(ks)
    walks = []
    for split in (True, False):
        w = K().walk_begin(tt, pp, nn, acc_stride=D + 1)
        # the root, then zeros (the output buffers come uninitialised from walk_begin)
        assert torch.equal(w["acc_tokens"][:, 0], tt[:, 0]) and not w["acc_tokens"][:, 1:].any()
        assert not w["acc_nodes"].any() and bool((w["acc_len"] == 1).all())
        for t in range(D):
            K().walk_rows(w, N)
            rows = torch.from_numpy(packed[np.minimum(np.arange(B), packed.shape[0] - 1)]).to(DEV)
            lg = (rows + torch.from_numpy(rng.standard_normal((B, V)).astype(np.float32) * 0.1).to(DEV)
                  if t == 0 else rows)
            K().walk_step(w, lg.contiguous(), tt, pp, nn, walk_step=t, seed=5, step=3, top_p=0.9, temperature=0.8,
                          split=split)
        walks.append(w)
        rng = np.random.default_rng(12)  # same perturbation for the second pass
        _walk_case(rng, B, ks, budget, V, True)
    for k in ("acc_tokens", "acc_nodes", "acc_len", "last_node", "correction"):
        assert torch.equal(walks[0][k], walks[1][k]), k


def test_sample_tokens_full_vocab_and_counter_noise():
    g = torch.Generator(device="cpu").manual_seed(5)
    V = 152064
    x = (torch.randn(6, V, generator=g) * 2).to(torch.bfloat16).to(DEV)
    seq = torch.tensor([0, 5, 9, 100, 7, 3], dtype=torch.int32, device=DEV)
    for kw in [dict(), dict(top_p=0.95), dict(top_k=40, temperature=0.7)]:
        out = K().sample_tokens(x, seed=1234, step=17, seq_ids=seq, draw=2, **kw)
        xs = to_np(x)
        want = [OS.sample_row(xs[i], OS.counter_noise(1234, 17, int(seq[i]), 2), **kw) for i in range(6)]
        assert out.tolist() == want


def test_sampling_law_matches_reference_distribution_tests():
    # flashgrpo/tests/test_exact_acceptance_distribution.py:17-37 on the device sampler
    for i, (vals, top_p) in enumerate([([5.0, 4.0, 0.0, -1.0], 0.85), ([0.0, 0.0, 0.0, 0.0], 0.75)]):
        n = 50000
        x = torch.tensor(vals, dtype=torch.float32, device=DEV).reshape(1, 4).expand(n, 4).contiguous()
        # pad rows to a multiple-of-8 stride
        xp = torch.full((n, 8), -1e30, device=DEV)
        xp[:, :4] = x
        out = K().sample_tokens(xp[:, :4], seed=321 + i, temperature=0.8, top_p=top_p)
        obs = np.bincount(out.cpu().numpy(), minlength=4) / n
        exp = OS.logits_to_probs(np.array(vals), temperature=0.8, top_p=top_p)
        assert np.max(np.abs(obs - exp)) < 0.015


# ------------------------------------------------------------------ acceptance walk
def _walk_case(rng, B, ks, budget, V, planted):
    parents, depths, ranks = OT.dense_topology(ks, budget)
    N = len(parents)
    toks = rng.integers(0, V, (B, N)).astype(np.int32)
    trees = [OT.Tree(toks[b].tolist(), parents, depths) for b in range(B)]
    _, _, slots = OT.internal_slots(trees)
    R = sum(1 for s in slots for v in s if v >= 0)
    packed = rng.standard_normal((R, V)).astype(np.float32)
    if planted:
        for b, t in enumerate(trees):
            for n in range(N):
                kids = t.children(n)
                if kids and slots[b][n] >= 0:
                    packed[slots[b][n], t.tokens[kids[min(b % len(kids), len(kids) - 1)]]] += 12.0
    return trees, parents, N, slots, packed


@pytest.mark.parametrize("planted", [False, True])
@pytest.mark.parametrize("emit_correction", [False, True])
@pytest.mark.parametrize("mode", [dict(), dict(top_p=0.9), dict(greedy=True), dict(temperature=0.7, top_k=20)])
def test_accept_walk_bit_exact(planted, emit_correction, mode):
    rng = np.random.default_rng(7 + planted)
    B, ks, budget, V = 16, [4, 2, 1, 1], 32, 64
    trees, parents, N, slots, packed = _walk_case(rng, B, ks, budget, V, planted)
    D = len(ks)
    u, nz = noise_i32(B, D, 99)
    lg = torch.from_numpy(packed).to(DEV)
    tt = torch.tensor([t.tokens for t in trees], dtype=torch.int32, device=DEV)
    pp = torch.tensor([parents] * B, dtype=torch.int32, device=DEV)
    nn = torch.full((B,), N, dtype=torch.int32, device=DEV)
    sm = torch.tensor(slots, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    greedy = mode.get("greedy", False)
    w = K().accept_walk(lg, tt, pp, nn, max_walk_steps=D, slot_map=sm, noise=nz, temperature=mode.get("temperature", 1.0),
                        greedy=greedy, top_k=mode.get("top_k"), top_p=mode.get("top_p", 1.0), err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    res = OS.accept_walk(trees, packed, u.tolist(), do_sample=not greedy, temperature=mode.get("temperature", 1.0),
                         top_p=mode.get("top_p", 1.0), top_k=mode.get("top_k"), slots=slots, emit_correction=True)
    toks, nodes, last, corr = res
    L = w["acc_len"].tolist()
    for b in range(B):
        assert L[b] == len(toks[b])
        assert w["acc_tokens"][b, :L[b]].tolist() == toks[b]
        assert w["acc_nodes"][b, :L[b]].tolist() == nodes[b]
        assert int(w["last_node"][b]) == last[b]
        assert int(w["correction"][b]) == (-1 if corr[b] is None else corr[b])
    if planted:
        assert max(L) == D + 1


def test_accept_walk_dense_equals_packed_reference_case():
    import json
    import os

    c = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))["acceptance"]["packed"]
    dense = np.full((2, 4, 16), -10.0, np.float32)
    for h in c["hot"]:
        dense[h[0], h[1], h[2]] = 10.0
    packed = np.stack([dense[0, 0], dense[0, 1], dense[1, 0], dense[1, 2]])
    tt = torch.tensor([t["tokens"] for t in c["trees"]], dtype=torch.int32, device=DEV)
    pp = torch.tensor([t["parents"] for t in c["trees"]], dtype=torch.int32, device=DEV)
    nn = torch.full((2,), 4, dtype=torch.int32, device=DEV)
    pad = lambda a: torch.from_numpy(np.concatenate([a, np.full(a.shape[:-1] + (0,), 0, np.float32)], -1)).to(DEV)
    r1 = K().accept_walk(pad(dense.reshape(8, 16)), tt, pp, nn, max_walk_steps=2, greedy=True)
    r2 = K().accept_walk(pad(packed), tt, pp, nn, max_walk_steps=2, greedy=True,
                         slot_map=torch.tensor(c["slots"], dtype=torch.int32, device=DEV))
    for r in (r1, r2):
        L = r["acc_len"].tolist()
        assert [r["acc_tokens"][b, :L[b]].tolist() for b in range(2)] == c["expect_tokens"]
        assert [r["acc_nodes"][b, :L[b]].tolist() for b in range(2)] == c["expect_nodes"]
        assert r["last_node"].tolist() == c["expect_last"]


def test_accept_finalize_matches_oracle_clamp():
    rng = np.random.default_rng(1)
    B, W = 12, 5
    acc = rng.integers(0, 6, (B, W)).astype(np.int32)
    nodes = np.tile(np.arange(W, dtype=np.int32), (B, 1))
    lens = rng.integers(1, W + 1, B).astype(np.int32)
    corr = rng.integers(-1, 6, B).astype(np.int32)
    old = rng.integers(90, 101, B).astype(np.int32)
    walk = dict(acc_tokens=torch.from_numpy(acc).to(DEV), acc_nodes=torch.from_numpy(nodes).to(DEV),
                acc_len=torch.from_numpy(lens.copy()).to(DEV), last_node=torch.zeros(B, dtype=torch.int32, device=DEV),
                correction=torch.from_numpy(corr).to(DEV))
    pend = torch.empty(B, dtype=torch.int32, device=DEV)
    fin = K().accept_finalize(walk, torch.from_numpy(old).to(DEV), max_length=100, eos_token_id=2, pending_root=pend)
    torch.cuda.synchronize()
    for b in range(B):
        t, n, f, _ = OS.clamp_accepted(acc[b, :lens[b]].tolist(), nodes[b, :lens[b]].tolist(), remaining=100 - old[b],
                                       eos_token_id=2, old_len=old[b], max_length=100)
        assert int(walk["acc_len"][b]) == len(t) and bool(fin[b]) == f
        assert int(walk["last_node"][b]) == n[-1]
        want_p = corr[b] if (corr[b] >= 0 and len(t) == lens[b] and not f) else -1
        assert int(pend[b]) == want_p


# ------------------------------------------------------------------ contractions
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,Kd", [(1, 1000, 128), (64, 4096, 512), (65, 1024, 256), (200, 3000, 512),
                                    (300, 512, 1536)])
def test_lm_head_matches_fp32_reference(dtype, M, N, Kd):
    torch.manual_seed(M + N)
    x = (torch.randn(M + 7, Kd, device=DEV) * 0.5).to(dtype)
    w = (torch.randn(N, Kd, device=DEV) * 0.05).to(dtype)
    idx = torch.randperm(M + 7, device=DEV)[:M].to(torch.int32)
    out = K().lm_head(x, w, row_index=idx, out_dtype=torch.float32)
    ref = x.float()[idx.long()] @ w.float().t()
    assert rel_err(to_np(out), to_np(ref)) < TOL[dtype]
    out2 = K().lm_head(x, w)
    assert rel_err(to_np(out2), to_np(x.float() @ w.float().t())) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_medusa_heads_match_oracle(dtype):
    rng = np.random.default_rng(2)
    B, H, nh = 16, 512, 3
    heads = OM.random_medusa(H, nh, seed=4, std=0.05)
    heads[1]["ln_w"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    heads[1]["ln_b"] = (0.1 * rng.standard_normal(H)).astype(np.float32)
    h = rng.standard_normal((B, H)).astype(np.float32)
    hd = torch.from_numpy(h).to(DEV).to(dtype)
    out = K().medusa_heads(hd, torch.from_numpy(np.stack([x["ln_w"] for x in heads])).to(DEV),
                           torch.from_numpy(np.stack([x["ln_b"] for x in heads])).to(DEV),
                           torch.from_numpy(np.stack([x["fc_w"] for x in heads])).to(DEV).to(dtype),
                           torch.from_numpy(np.stack([x["fc_b"] for x in heads])).to(DEV).to(dtype),
                           out_dtype=torch.float32)
    hs = to_np(hd)
    for i, hp in enumerate(heads):
        hp = dict(hp, fc_w=to_np(torch.from_numpy(hp["fc_w"]).to(dtype)), fc_b=to_np(torch.from_numpy(hp["fc_b"]).to(dtype)))
        want = OM.medusa_project(hs, hp)
        assert rel_err(to_np(out[i * B:(i + 1) * B]), want) < TOL[dtype]


@pytest.mark.parametrize("B,H,nh", [(96, 4096, 1), (64, 3584, 4), (7, 516, 2), (130, 256, 3)])
def test_medusa_heads_fp32_split_matches_float64(B, H, nh):
    """fp32 Medusa blocks (the chain path's head-0 bootstrap with fp32 master weights: 96 rows x
    4096 at the Llama-3.1-8B shape) run split over K into parts that a combine kernel sums in order
    with the bias, SiLU and residual. Checked against float64 on the normalised rows the call
    wrote, within the fp32 accumulation bound, for hidden sizes that are not multiples of 64 (516)
    and row counts past one 64-row tile; repeated calls give identical bits."""
    torch.manual_seed(B + H + nh)
    hid = torch.randn(B + 2, H, device=DEV)[:B]
    ln_w = 1 + 0.1 * torch.randn(nh, H, device=DEV)
    ln_b = 0.1 * torch.randn(nh, H, device=DEV)
    fc_w = torch.randn(nh, H, H, device=DEV) * 0.03
    fc_b = torch.randn(nh, H, device=DEV) * 0.1
    need = K()._lib.load().fg_medusa_heads_workspace(B, H, nh, 0)
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    out = K().medusa_heads(hid, ln_w, ln_b, fc_w, fc_b, out_dtype=torch.float32, workspace=ws)
    rows = ws[:nh * B * H * 4].view(torch.float32).view(nh, B, H).double()
    pre = torch.bmm(rows, fc_w.double().transpose(1, 2).contiguous()) + fc_b.double()[:, None, :]
    ref = hid.double()[None] + torch.nn.functional.silu(pre)
    # fp32 sums of H products (split parts plus their in-order sum), SiLU' <= 1.1
    bound = 1.1 * (H + 16) * 2.0 ** -24 * (torch.bmm(rows.abs(), fc_w.double().abs().transpose(1, 2).contiguous())
                                           + fc_b.double().abs()[:, None, :]) + 4 * 2.0 ** -24 * ref.abs() + 1e-30
    err = (out.view(nh, B, H).double() - ref).abs()
    assert bool((err <= bound).all()), float((err - bound).max())
    ln = torch.nn.functional.layer_norm(hid.double(), (H,), eps=1e-5)
    assert rel_err(to_np(rows), to_np(ln[None] * ln_w.double()[:, None, :] + ln_b.double()[:, None, :])) < 1e-5
    again = K().medusa_heads(hid, ln_w, ln_b, fc_w, fc_b, out_dtype=torch.float32, workspace=ws)
    assert torch.equal(out, again)


@pytest.mark.parametrize("B,H,nh", [(64, 3584, 4), (16, 576, 3), (100, 1024, 5), (200, 512, 2), (1, 128, 1)])
def test_medusa_heads_stream_matches_fp32_reference(B, H, nh):
    """bf16 Medusa fc through the weight stream (key ranges summed by a second launch):
    the normalised rows are read back from the workspace the call used, and
    hidden + SiLU(rows . fc_w^T + fc_b) is recomputed in fp32 from them. Shapes cover the
    Qwen2.5-7B block (4 heads x 3584, 64 rows), a last 256-column group that is partly
    empty (576), 65-128 and 129-256 rows, and one row of one head. Repeated calls give
    identical bits (the ranges are added in a fixed order)."""
    torch.manual_seed(B * 7 + H)
    dt = torch.bfloat16
    hid = torch.randn(B + 3, H, device=DEV).to(dt)[:B]
    ln_w = 1 + 0.1 * torch.randn(nh, H, device=DEV)
    ln_b = 0.1 * torch.randn(nh, H, device=DEV)
    fc_w = (torch.randn(nh, H, H, device=DEV) * 0.03).to(dt)
    fc_b = (torch.randn(nh, H, device=DEV) * 0.1).to(dt)
    need = K()._lib.load().fg_medusa_heads_workspace(B, H, nh, 1)
    assert need >= nh * B * H * 2 + 256
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    out = K().medusa_heads(hid, ln_w, ln_b, fc_w, fc_b, out_dtype=torch.float32, workspace=ws)
    rows = ws[:nh * B * H * 2].view(dt).view(nh, B, H).float()
    ref = torch.bmm(rows, fc_w.float().transpose(1, 2).contiguous()) + fc_b.float()[:, None, :]
    ref = hid.float()[None] + torch.nn.functional.silu(ref)
    assert rel_err(to_np(out.view(nh, B, H)), to_np(ref)) < 1e-5
    # the normalised rows themselves against LayerNorm in fp32 (bf16 rounding of the output)
    ln = torch.nn.functional.layer_norm(hid.float(), (H,), eps=1e-5)
    ln_ref = ln[None] * ln_w[:, None, :] + ln_b[:, None, :]
    assert rel_err(to_np(rows), to_np(ln_ref)) < 1e-2
    out_bf = K().medusa_heads(hid, ln_w, ln_b, fc_w, fc_b, workspace=ws)
    assert out_bf.dtype == dt
    # bf16 output: rounded where the reference's bf16 head rounds (fc + bias, SiLU, the sum); the
    # emulation's fc sums run in the library's order, so a rounding tie may fall the other way
    pre = torch.bmm(rows, fc_w.float().transpose(1, 2).contiguous()) + fc_b.float()[:, None, :]
    emu = (hid.float()[None] + torch.nn.functional.silu(pre.to(dt).float()).to(dt).float()).to(dt)
    same = float((out_bf.view(nh, B, H).view(torch.int16) == emu.view(torch.int16)).float().mean())
    assert same >= 0.98, same
    assert rel_err(to_np(out_bf), to_np(out)) < 2e-2
    again = K().medusa_heads(hid, ln_w, ln_b, fc_w, fc_b, out_dtype=torch.float32, workspace=ws)
    assert torch.equal(again, out)


# ------------------------------------------------------------------ attention and layer pieces
def _attn_reference(q, kc, vc, seq, anc, N, G):
    B, _, Hq, d = q.shape
    out = np.zeros_like(q, dtype=np.float64)
    for b in range(B):
        for n in range(N):
            for hq in range(Hq):
                hk = hq // G
                s0 = seq[b]
                keys = list(range(s0)) + [s0 + m for m in range(N) if (int(anc[b][n]) >> m) & 1]
                kk = kc[b, hk, keys].astype(np.float64)
                vv = vc[b, hk, keys].astype(np.float64)
                s = kk @ q[b, n, hq].astype(np.float64) / np.sqrt(d)
                p = np.exp(s - s.max())
                out[b, n, hq] = (p / p.sum()) @ vv
    return out


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 64), (torch.float32, 128)])
@pytest.mark.parametrize("ks,budget,Hq,Hkv", [([4, 2, 1, 1], 32, 28, 4), ([4, 2], 16, 8, 2), ([3], 4, 12, 2),
                                               ([1] * 63, 64, 4, 1), ([2] * 5, 48, 28, 4)])
def test_tree_attention_matches_reference(dtype, d, ks, budget, Hq, Hkv):
    rng = np.random.default_rng(len(ks) + Hq)
    parents, depths, _ = OT.dense_topology(ks, budget)
    N = len(parents)
    B, S = 3, 300
    seq = np.array([0, 37, 200], np.int32)[:B] if N < 64 else np.array([5, 100, 230], np.int32)
    anc_bits = OT.ancestor_bits(parents)
    anc = np.array([anc_bits] * B, dtype=np.uint64)
    q = rng.standard_normal((B, N, Hq, d)).astype(np.float32)
    kc = rng.standard_normal((B, Hkv, S, d)).astype(np.float32)
    vc = rng.standard_normal((B, Hkv, S, d)).astype(np.float32)
    qt = torch.from_numpy(q).to(DEV).to(dtype)
    kt = torch.from_numpy(kc).to(DEV).to(dtype)
    vt = torch.from_numpy(vc).to(DEV).to(dtype)
    anct = torch.from_numpy(anc.view(np.int64)).to(DEV)
    out = K().tree_attention(qt, kt, vt, seq_len=torch.from_numpy(seq).to(DEV), anc=anct, num_nodes=N, q_heads=Hq,
                             kv_heads=Hkv, head_dim=d)
    want = _attn_reference(to_np(qt), to_np(kt), to_np(vt), seq, anc, N, Hq // Hkv)
    assert rel_err(to_np(out), want) < TOL[dtype]


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_tree_attention_causal_chain(dtype, d):
    """No masks (anc None): new token n sees the prefix and new tokens 0..n. Equals the
    explicit chain masks bit for bit at 64 tokens, and the reference beyond 64 (prefill
    chunks), with ragged prefixes and GQA."""
    rng = np.random.default_rng(17)
    Hq, Hkv = 8, 2
    for N, seq in ((64, [0, 40, 150]), (300, [0, 77, 5]), (257, [130, 0, 64])):
        B, S = 3, 520
        seq = np.array(seq, np.int32)
        q = torch.from_numpy(rng.standard_normal((B, N, Hq, d)).astype(np.float32)).to(DEV).to(dtype)
        kt = torch.from_numpy(rng.standard_normal((B, Hkv, S, d)).astype(np.float32)).to(DEV).to(dtype)
        vt = torch.from_numpy(rng.standard_normal((B, Hkv, S, d)).astype(np.float32)).to(DEV).to(dtype)
        sl = torch.from_numpy(seq).to(DEV)
        out = K().tree_attention(q, kt, vt, seq_len=sl, anc=None, num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=d)
        if N <= 64:
            bits = [(1 << (n + 1)) - 1 for n in range(N)]
            anc = torch.from_numpy(np.array(bits, dtype=np.uint64).view(np.int64)).to(DEV)
            masked = K().tree_attention(q, kt, vt, seq_len=sl, anc=anc, num_nodes=N, q_heads=Hq, kv_heads=Hkv,
                                        head_dim=d)
            assert torch.equal(out, masked)
        qs, ks_, vs = to_np(q), to_np(kt), to_np(vt)
        for b in range(B):
            for n in (0, 1, N // 2, N - 1):
                for hq in (0, 5):
                    keys = list(range(seq[b] + n + 1))
                    kk = ks_[b, hq // (Hq // Hkv), keys].astype(np.float64)
                    vv = vs[b, hq // (Hq // Hkv), keys].astype(np.float64)
                    sc = kk @ qs[b, n, hq].astype(np.float64) / np.sqrt(d)
                    p = np.exp(sc - sc.max())
                    want = (p / p.sum()) @ vv
                    assert rel_err(to_np(out[b, n, hq]), want) < TOL[dtype], (N, b, n, hq)


@pytest.mark.parametrize("ks,budget,Hq,Hkv", [([4, 2, 1, 1], 32, 28, 4), ([2] * 5, 48, 12, 2), ([1] * 63, 64, 4, 1)])
def test_tree_attention_key_split(ks, budget, Hq, Hkv):
    """Few sequences and a long cache: keys are split over several workgroups (with
    empty parts for short rows) and merged by the combine launch."""
    from flashgrpo_amd import _lib

    rng = np.random.default_rng(Hq + len(ks))
    parents, depths, _ = OT.dense_topology(ks, budget)
    N = len(parents)
    B, S, d = 3, 1100, 128
    seq = np.array([0, 333, 1100 - 64], np.int32)
    assert _lib.load().fg_tree_attention_workspace(B, N, Hq, Hkv, d, S) > 0  # the split path runs
    anc = np.array([OT.ancestor_bits(parents)] * B, dtype=np.uint64)
    q = torch.from_numpy(rng.standard_normal((B, N, Hq, d)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    kt = torch.from_numpy(rng.standard_normal((B, Hkv, S, d)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    vt = torch.from_numpy(rng.standard_normal((B, Hkv, S, d)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    anct = torch.from_numpy(anc.view(np.int64)).to(DEV)
    out = K().tree_attention(q, kt, vt, seq_len=torch.from_numpy(seq).to(DEV), anc=anct, num_nodes=N, q_heads=Hq,
                             kv_heads=Hkv, head_dim=d)
    want = _attn_reference(to_np(q), to_np(kt), to_np(vt), seq, anc, N, Hq // Hkv)
    assert rel_err(to_np(out), want) < TOL[torch.bfloat16]


@pytest.mark.parametrize("B,half,ks,budget,Hq,Hkv,S", [(64, 32, [4, 2, 1, 1], 32, 28, 4, 900),
                                                       (16, 8, [4, 3, 2, 1], 64, 40, 8, 300)])
def test_tree_attention_wave_layouts_agree(B, half, ks, budget, Hq, Hkv, S):
    """A batch that fills the chip runs 8-wave workgroups (one or two row tiles per KV
    head); half of it runs 4-wave workgroups, two per CU (two or three row tiles). Neither
    splits the keys, so every row sums the same terms in the same order: the half batch
    equals the first rows of the full batch bit for bit, and sampled rows match the
    reference."""
    from flashgrpo_amd import _lib

    rng = np.random.default_rng(B + Hq)
    parents, depths, _ = OT.dense_topology(ks, budget)
    N = len(parents)
    lib = _lib.load()
    assert lib.fg_tree_attention_workspace(B, N, Hq, Hkv, 128, S) == 0
    assert lib.fg_tree_attention_workspace(half, N, Hq, Hkv, 128, S) == 0
    seq = rng.integers(0, S - N + 1, B).astype(np.int32)
    seq[:3] = [0, S - N, 1]
    anc = np.array([OT.ancestor_bits(parents)] * B, dtype=np.uint64)
    q = torch.from_numpy(rng.standard_normal((B, N, Hq, 128)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    kt = torch.from_numpy(rng.standard_normal((B, Hkv, S, 128)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    vt = torch.from_numpy(rng.standard_normal((B, Hkv, S, 128)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    anct = torch.from_numpy(anc.view(np.int64)).to(DEV)
    sl = torch.from_numpy(seq).to(DEV)
    kw = dict(num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=128)
    full = K().tree_attention(q, kt, vt, seq_len=sl, anc=anct, **kw)
    part = K().tree_attention(q[:half].contiguous(), kt[:half].contiguous(), vt[:half].contiguous(),
                              seq_len=sl[:half].contiguous(), anc=anct[:half].contiguous(), **kw)
    assert torch.equal(full[:half], part)
    qs, ks_, vs = to_np(q), to_np(kt), to_np(vt)
    G = Hq // Hkv
    for b in (0, 1, 2, half, B - 1):
        for n in (0, N // 2, N - 1):
            for hq in (0, Hq - 1):
                keys = list(range(seq[b])) + [seq[b] + m for m in range(N) if (int(anc[b][n]) >> m) & 1]
                kk = ks_[b, hq // G, keys].astype(np.float64)
                vv = vs[b, hq // G, keys].astype(np.float64)
                sc = kk @ qs[b, n, hq].astype(np.float64) / np.sqrt(128)
                p = np.exp(sc - sc.max())
                assert rel_err(to_np(full[b, n, hq]), (p / p.sum()) @ vv) < TOL[torch.bfloat16], (b, n, hq)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_kv_write_rmsnorm_swiglu(dtype):
    rng = np.random.default_rng(9)
    B, N, Hq, Hkv, d, S = 3, 5, 4, 2, 64, 50
    seq = np.array([0, 7, 30], np.int32)
    pos_off = np.array([0, 1, 1, 2, 2], np.int32)
    inv = OM.inv_freq_table(d, 1e6)
    qkv = rng.standard_normal((B * N, (Hq + 2 * Hkv) * d)).astype(np.float32)
    qkvd = torch.from_numpy(qkv).to(DEV).to(dtype)
    qo = torch.empty(B, N, Hq, d, dtype=dtype, device=DEV)
    kc = torch.zeros(B, Hkv, S, d, dtype=dtype, device=DEV)
    vc = torch.zeros(B, Hkv, S, d, dtype=dtype, device=DEV)
    K().rope_kv_write(qkvd, batch=B, num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=d,
                      seq_len=torch.from_numpy(seq).to(DEV), pos_offset=torch.from_numpy(pos_off).to(DEV),
                      inv_freq=torch.from_numpy(inv).to(DEV), q_out=qo, k_cache=kc, v_cache=vc)
    x = to_np(qkvd).reshape(B, N, Hq + 2 * Hkv, d)
    pos = seq[:, None] + pos_off[None]
    cos, sin = OM.rope_cos_sin(pos, inv)
    qr = OM.apply_rope(x[:, :, :Hq], cos[:, :, None], sin[:, :, None])
    kr = OM.apply_rope(x[:, :, Hq:Hq + Hkv], cos[:, :, None], sin[:, :, None])
    tol = TOL[dtype] if dtype == torch.bfloat16 else 2e-6
    assert rel_err(to_np(qo), qr) < tol
    for b in range(B):
        for n in range(N):
            assert rel_err(to_np(kc[b, :, seq[b] + n]), kr[b, n]) < tol
            assert np.array_equal(to_np(vc[b, :, seq[b] + n]), x[b, n, Hq + Hkv:])
    # rmsnorm with fused residual add
    H = 384
    xr = torch.from_numpy(rng.standard_normal((7, H)).astype(np.float32)).to(DEV).to(dtype)
    dl = torch.from_numpy(rng.standard_normal((7, H)).astype(np.float32)).to(DEV).to(dtype)
    w = torch.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)).to(DEV).to(dtype)
    summed = (xr.float() + dl.float()).to(dtype)
    y = K().rmsnorm(xr, w, 1e-6, delta=dl)
    assert torch.equal(xr, summed)
    assert rel_err(to_np(y), OM.rmsnorm(to_np(summed), to_np(w), 1e-6)) < TOL[dtype]
    gu = torch.from_numpy(rng.standard_normal((5, 2 * 96)).astype(np.float32)).to(DEV).to(dtype)
    sg = K().swiglu(gu)
    g_ = to_np(gu)
    assert rel_err(to_np(sg), OM.silu(g_[:, :96].astype(np.float64)) * g_[:, 96:]) < TOL[dtype]


@pytest.mark.parametrize("mode", [{}, {"temperature": 0.7}, {"greedy": True}, {"top_p": 0.9}])
def test_walk_with_lm_head_parts_equals_plain_walk(mode):
    """The lazy walk with the LM head's row maxima (no chunk-maxima launch in an
    unrestricted / greedy step, next rows written by the step) equals the walk with chunk maxima and
    fg_walk_rows, and the one-workgroup-per-row walk, step by step; planted logits make
    sequences accept several nodes."""
    rng = np.random.default_rng(5)
    B, ks, budget, V, H = 16, [4, 2, 1, 1], 32, 5003, 128
    parents, _, _ = OT.dense_topology(ks, budget)
    N, D = len(parents), len(ks)
    toks = rng.integers(0, V, (B, N)).astype(np.int32)
    trees = [OT.Tree(toks[b].tolist(), parents, None) for b in range(B)]
    w = torch.from_numpy(rng.standard_normal((V, H)).astype(np.float32) * 0.05).to(torch.bfloat16).to(DEV)
    hid = torch.from_numpy(rng.standard_normal((B * N, H)).astype(np.float32) * 0.5)
    wf = w.float().cpu()
    for b, t in enumerate(trees):  # steer most internal nodes toward one of their children
        for n in range(N):
            kids = t.children(n)
            if kids and (b + n) % 4:
                tok = t.tokens[kids[(b + n) % len(kids)]]
                hid[b * N + n] = wf[tok] * (14.0 / float(wf[tok].pow(2).sum()))
    hid = hid.to(torch.bfloat16).to(DEV)
    tt = torch.from_numpy(toks).to(DEV)
    pp = torch.tensor([parents] * B, dtype=torch.int32, device=DEV)
    nn = torch.full((B,), N, dtype=torch.int32, device=DEV)
    P = K().lm_head_parts(V)
    kw = dict(seed=3, step=2, temperature=mode.get("temperature", 1.0), greedy=mode.get("greedy", False),
              top_p=mode.get("top_p", 1.0))
    runs = []
    for variant in ("parts", "split", "single"):
        wk = K().walk_begin(tt, pp, nn, acc_stride=D + 1)
        parts = (torch.empty(B, P, dtype=torch.float32, device=DEV), torch.empty(B, P, dtype=torch.int64, device=DEV))
        steps = []
        K().walk_rows(wk, N)
        for t in range(D):
            if variant != "parts" and t > 0:
                K().walk_rows(wk, N)
            lg = torch.full((B, V), 5.0, dtype=torch.bfloat16, device=DEV)
            K().lm_head_topk(hid, w, 0, row_index=wk["row_index"], row_active=wk["row_active"], out=lg,
                             parts=parts if variant == "parts" else None)
            K().walk_step(wk, lg, tt, pp, nn, walk_step=t, split=variant != "single",
                          parts=parts if variant == "parts" else None, next_rows=variant == "parts", **kw)
            steps.append(wk["state"][: 3 * B].clone())
        runs.append((wk, steps))
    for wk, steps in runs[1:]:
        for k in ("acc_tokens", "acc_nodes", "acc_len", "last_node", "correction"):
            assert torch.equal(runs[0][0][k], wk[k]), k
        for t in range(D):
            assert torch.equal(runs[0][1][t], steps[t]), t
    assert int(runs[0][0]["acc_len"].max()) >= 3  # the planted paths were walked


@pytest.mark.parametrize("mode", [{}, {"temperature": 0.7}, {"top_p": 0.9}, {"greedy": True}])
def test_planted_deep_lazy_walk_full_vocab_matches_oracle(mode):
    """The lazy walk at the 7B configuration's vocabulary, batch and tree (V = 152064, 64
    sequences, [4, 2, 1, 1] in 32 nodes) against ``oracle.sampling.accept_walk``: hidden
    rows steer four of every five internal nodes to one of their children, so most
    sequences accept deep paths; each step projects the rows the walk stands on with the
    weight-streaming LM head (row maxima parts, next rows written by the step) and draws
    with ``fg_walk_step`` under counter noise. The oracle walks the same trees on the
    device's logits rows (checked against an fp32 product) with the same noise; accepted
    tokens, nodes, lengths, last nodes and correction tokens are equal."""
    rng = np.random.default_rng(11)
    B, ks, budget, V, H = 64, [4, 2, 1, 1], 32, 152064, 256
    parents, _, _ = OT.dense_topology(ks, budget)
    N, D = len(parents), len(ks)
    toks = rng.integers(0, V, (B, N)).astype(np.int32)
    trees = [OT.Tree(toks[b].tolist(), parents, None) for b in range(B)]
    g = torch.Generator(device="cpu").manual_seed(5)
    w = (torch.randn(V, H, generator=g) * 0.05).to(torch.bfloat16)
    hid = torch.from_numpy(rng.standard_normal((B * N, H)).astype(np.float32) * 0.5)
    wf = w.float()
    for b, t in enumerate(trees):
        for n in range(N):
            kids = t.children(n)
            if kids and (b + n) % 5:
                tok = t.tokens[kids[(b + n) % len(kids)]]
                hid[b * N + n] = wf[tok] * (24.0 / float(wf[tok].pow(2).sum()))
    hid, w = hid.to(torch.bfloat16).to(DEV), w.to(DEV)
    tt = torch.from_numpy(toks).to(DEV)
    pp = torch.tensor([parents] * B, dtype=torch.int32, device=DEV)
    nn = torch.full((B,), N, dtype=torch.int32, device=DEV)
    P = K().lm_head_parts(V)
    parts = (torch.empty(B, P, dtype=torch.float32, device=DEV), torch.empty(B, P, dtype=torch.int64, device=DEV))
    T, greedy, top_p = mode.get("temperature", 1.0), mode.get("greedy", False), mode.get("top_p", 1.0)
    wk = K().walk_begin(tt, pp, nn, acc_stride=D + 1)
    K().walk_rows(wk, N)
    step_logits = []
    for t in range(D):
        lg = torch.full((B, V), 5.0, dtype=torch.bfloat16, device=DEV)
        K().lm_head_topk(hid, w, 0, row_index=wk["row_index"], row_active=wk["row_active"], out=lg, parts=parts)
        K().walk_step(wk, lg, tt, pp, nn, walk_step=t, seed=3, step=2, temperature=T, greedy=greedy, top_p=top_p,
                      parts=parts, next_rows=True)
        step_logits.append(lg)
    torch.cuda.synchronize()
    acc_len = wk["acc_len"].cpu().numpy()
    acc_nodes = wk["acc_nodes"].cpu().numpy()
    # the rows each sequence sampled from, packed; nodes the device never stood on map to a
    # trailing zero row (a walk that left the device's path would read it and mismatch)
    visited = [(b, t, int(acc_nodes[b, t])) for b in range(B) for t in range(int(acc_len[b]))
               if trees[b].children(int(acc_nodes[b, t]))]
    packed = np.zeros((len(visited) + 1, V), np.float32)
    slots = [[len(visited)] * N for _ in range(B)]
    for j, (b, t, node) in enumerate(visited):
        packed[j] = to_np(step_logits[t][b])
        slots[b][node] = j
    rows = torch.tensor([b * N + node for b, _, node in visited], device=DEV)
    want_lg = to_np(hid[rows].float() @ w.float().t())
    assert rel_err(packed[:-1], want_lg) < 2e-2
    nz = [[OS.counter_noise(3, 2, b, 1 + t) for t in range(D)] for b in range(B)]
    at, an, last, corr = OS.accept_walk(trees, packed, nz, do_sample=not greedy, temperature=T, top_p=top_p,
                                        top_k=None, slots=slots, emit_correction=True)
    for b in range(B):
        L = int(acc_len[b])
        assert L == len(at[b]), b
        assert wk["acc_tokens"][b, :L].tolist() == at[b], b
        assert acc_nodes[b, :L].tolist() == an[b], b
        assert int(wk["last_node"][b]) == last[b], b
        assert int(wk["correction"][b]) == (-1 if corr[b] is None else corr[b]), b
    assert int(acc_len.max()) == D + 1 and int((acc_len == D + 1).sum()) >= B // 4
