"""The weight-streaming LM head with the fused per-row top-k (``fg_lm_head_topk``).

Logits are checked against an fp32 product; the candidates, scores and (max, logsumexp)
against ``oracle.tree.topk_canonical`` / ``nan_to_num_logits`` applied to the kernel's own
bf16 logits (the values the reference ranks, medusa_tree.py:239-252), so the epilogue is
pinned bit for bit independently of the GEMM's rounding.
"""
import numpy as np
import pytest
import torch

from oracle import tree as OT

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from flashgrpo_amd import _lib

    _lib.load()


def K():
    from flashgrpo_amd import kernels

    return kernels


def to_np(t):
    return t.detach().float().cpu().numpy()


def rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def check_candidates(lg, tok, sc, st, kmax, sanitize):
    xs = to_np(lg)
    for r in range(xs.shape[0]):
        row = OT.nan_to_num_logits(xs[r]) if sanitize else xs[r]
        ids, vals = OT.topk_canonical(row, kmax)
        assert tok[r].tolist() == ids.tolist(), r
        assert np.array_equal(to_np(sc[r]), vals.astype(np.float32) + 0.0, equal_nan=True), r
        if st is not None and np.all(np.isfinite(row)):
            m = float(row.max())
            lse = np.log(np.sum(np.exp(row.astype(np.float64) - m))) + m
            assert float(st[r, 0]) == m, r
            assert abs(float(st[r, 1]) - lse) < 1e-4 * max(1.0, abs(lse)), r


@pytest.mark.parametrize("M,N,Kd", [(1, 1000, 64), (33, 4099, 512), (64, 32000, 256), (100, 5003, 512),
                                    (192, 8192, 128), (256, 3000, 512)])
def test_logits_match_fp32(M, N, Kd):
    torch.manual_seed(M + N)
    x = (torch.randn(M, Kd, device=DEV) * 0.5).to(torch.bfloat16)
    w = (torch.randn(N, Kd, device=DEV) * 0.05).to(torch.bfloat16)
    ref = to_np(x.float() @ w.float().t())
    lg, tok, sc, st = K().lm_head_topk(x, w, 0)
    assert tok is None and sc is None and st is None
    assert rel_err(to_np(lg), ref) < 2e-2
    lg32 = K().lm_head_topk(x, w, 0, out_dtype=torch.float32)[0]
    assert lg32.dtype == torch.float32 and rel_err(to_np(lg32), ref) < 1e-5
    # a strided output view and gathered rows
    big = torch.full((M, N + 24), 7.0, dtype=torch.bfloat16, device=DEV)
    K().lm_head_topk(x, w, 0, out=big[:, :N])
    assert torch.equal(big[:, :N], lg) and bool((big[:, N:] == 7.0).all())
    src = (torch.randn(M + 9, Kd, device=DEV) * 0.5).to(torch.bfloat16)
    idx = torch.randperm(M + 9, device=DEV)[:M].to(torch.int32)
    g = K().lm_head_topk(src, w, 0, row_index=idx)[0]
    assert rel_err(to_np(g), to_np(src.float()[idx.long()] @ w.float().t())) < 2e-2


@pytest.mark.parametrize("M,N,kmax", [(64, 32000, 1), (64, 32000, 2), (37, 4099, 4), (128, 20000, 7),
                                      (192, 152064, 8), (100, 10000, 10), (64, 5000, 16), (256, 9000, 8),
                                      (3, 40, 16)])
@pytest.mark.parametrize("sanitize", [False, True])
def test_candidates_equal_canonical_topk(M, N, kmax, sanitize):
    g = torch.Generator(device="cpu").manual_seed(M * 7 + kmax)
    Kd = 128
    # quantised operands: many rows with exactly tied logits
    x = torch.randint(-3, 4, (M, Kd), generator=g).float()
    w = torch.randint(-2, 3, (N, Kd), generator=g).float() * 0.125
    x[: M // 3] = torch.randn(M // 3, Kd, generator=g)
    xd, wd = x.to(torch.bfloat16).to(DEV), w.to(torch.bfloat16).to(DEV)
    lg, tok, sc, st = K().lm_head_topk(xd, wd, kmax, stats=True, sanitize=sanitize)
    check_candidates(lg, tok, sc, st, kmax, sanitize)
    # without the logits: the same candidates
    none, tok2, sc2, st2 = K().lm_head_topk(xd, wd, kmax, logits=False, stats=True, sanitize=sanitize)
    assert none is None
    assert torch.equal(tok, tok2) and torch.equal(sc, sc2) and torch.equal(st, st2)
    # and equal to the stand-alone top-k over these logits
    t3, s3, st3 = K().medusa_topk(lg, kmax, stats=True, sanitize=sanitize)
    assert torch.equal(tok, t3) and torch.equal(sc, s3)
    assert float((st - st3).abs().max()) < 1e-4


@pytest.mark.parametrize("sanitize", [False, True])
def test_candidates_with_nan_and_inf_logits(sanitize):
    torch.manual_seed(3)
    M, N, Kd, kmax = 40, 3001, 64, 4
    x = (torch.randn(M, Kd, device=DEV)).to(torch.bfloat16)
    x[5, 7] = 0.0
    w = (torch.randn(N, Kd, device=DEV) * 0.1).to(torch.bfloat16)
    w[11, 7] = float("inf")     # +-inf logits, NaN in row 5 (0 * inf)
    w[2900, 3] = float("nan")   # NaN column
    w[1500, :] = -1.0e38
    lg, tok, sc, _ = K().lm_head_topk(x, w, kmax, stats=False, sanitize=sanitize)
    xs = to_np(lg)
    assert np.isnan(xs[:, 2900]).all() and np.isnan(xs[5, 11])
    check_candidates(lg, tok, sc, None, kmax, sanitize)


def test_repeated_calls_are_identical():
    torch.manual_seed(9)
    for M in (64, 128, 192):
        x = (torch.randn(M, 512, device=DEV)).to(torch.bfloat16)
        w = (torch.randn(40000, 512, device=DEV) * 0.05).to(torch.bfloat16)
        outs = [K().lm_head_topk(x, w, 16 if M <= 192 else 8, stats=True) for _ in range(3)]
        for o in outs[1:]:
            for a, b in zip(outs[0], o):
                assert torch.equal(a, b)


def test_row_active_skips_launch():
    x = torch.randn(8, 64, device=DEV).to(torch.bfloat16)
    w = torch.randn(500, 64, device=DEV).to(torch.bfloat16)
    out = torch.full((8, 500), 3.0, dtype=torch.bfloat16, device=DEV)
    K().lm_head_topk(x, w, 0, out=out, row_active=torch.zeros(8, dtype=torch.int32, device=DEV))
    assert bool((out == 3.0).all())
    act = torch.zeros(8, dtype=torch.int32, device=DEV)
    act[6] = 1
    K().lm_head_topk(x, w, 0, out=out, row_active=act)
    # the active row is written, the others keep their contents
    assert rel_err(to_np(out[6]), to_np(x[6].float() @ w.float().t())) < 2e-2
    assert bool((out[:6] == 3.0).all()) and bool((out[7:] == 3.0).all())


def test_target_logits_masked_writes_active_rows_only():
    from flashgrpo_amd.models.target import TargetModel, TargetConfig

    for dtype in (torch.bfloat16, torch.float32):
        cfg = TargetConfig(num_layers=1, hidden=128, q_heads=2, kv_heads=1, head_dim=64, intermediate=256, vocab=3001)
        model = TargetModel.random(cfg, seed=2, dtype=dtype, device=DEV)
        h = torch.randn(20, 128, device=DEV).to(dtype)
        out = torch.full((20, 3001), 5.0, dtype=dtype, device=DEV)
        act = torch.zeros(20, dtype=torch.int32, device=DEV)
        act[[1, 7, 19]] = 1
        model.logits_masked(h, act, out)
        full = model.logits(h)
        rows = act.bool()
        assert torch.equal(out[rows], full[rows]), dtype
        assert bool((out[~rows] == 5.0).all()), dtype
        model.logits_masked(h, torch.zeros_like(act), out)  # no active row: nothing changes
        assert torch.equal(out[rows], full[rows]) and bool((out[~rows] == 5.0).all())


def test_rejects_unsupported_shapes():
    from flashgrpo_amd._lib import NativeError

    errs = (ValueError, NativeError)

    w = torch.randn(1000, 128, device=DEV).to(torch.bfloat16)
    with pytest.raises(errs, match="M must be in"):
        K().lm_head_topk(torch.randn(257, 128, device=DEV).to(torch.bfloat16), w, 0)
    with pytest.raises(errs, match="multiple of 64"):
        K().lm_head_topk(torch.randn(4, 96, device=DEV).to(torch.bfloat16), torch.randn(10, 96, device=DEV).to(
            torch.bfloat16), 0)
    with pytest.raises(errs, match="kmax above 8"):
        K().lm_head_topk(torch.randn(200, 128, device=DEV).to(torch.bfloat16), w, 12)
    with pytest.raises(TypeError):
        K().lm_head_topk(torch.randn(4, 128, device=DEV), w, 0)


def test_target_lm_head_routes_hidden_96():
    """A bf16 target whose hidden size is not a multiple of 64 (96) runs every LM-head
    route on the library GEMM (the hand-written kernels take K % 64 == 0 only): contiguous,
    gathered and masked rows, the top-k path and the walk's row-maxima parts (None)."""
    from flashgrpo_amd.models.target import TargetModel, TargetConfig

    cfg = TargetConfig(num_layers=1, hidden=96, q_heads=1, kv_heads=1, head_dim=96, intermediate=192, vocab=3001)
    model = TargetModel.random(cfg, seed=4, dtype=torch.bfloat16, device=DEV)
    w = model.w["lm_head"]
    h = torch.randn(20, 96, device=DEV).to(torch.bfloat16)
    ref = (h.float() @ w.float().t())
    full = model.logits(h)
    assert full.shape == (20, 3001) and rel_err(to_np(full), to_np(ref)) < 2e-2
    idx = torch.tensor([3, 3, 0, 19], dtype=torch.int32, device=DEV)
    g = model.logits(h, row_index=idx)
    assert torch.equal(g, full[idx.long()])
    act = torch.zeros(20, dtype=torch.int32, device=DEV)
    act[[2, 5]] = 1
    out = torch.full((20, 3001), 7.0, dtype=torch.bfloat16, device=DEV)
    model.logits_masked(h, act, out)
    assert torch.equal(out[act.bool()], full[act.bool()]) and bool((out[~act.bool()] == 7.0).all())
    lg, tok, sc, st = model.logits_topk(h, 4, stats=True, logits=True)
    assert torch.equal(lg, full)
    check_candidates(lg, tok, sc, st, 4, False)
    assert model.walk_parts(20, h) is None


def test_target_logits_gathers_large_blocks_into_one_gemm():
    """Gathered bf16 rows above 256 (the packed tree's internal nodes) are gathered and
    projected by one GEMM: equal to the contiguous projection of the same rows, within bf16
    of an fp32 product, also into a given out; with row_active they stay on fg_lm_head (its
    active rows checked)."""
    from flashgrpo_amd.models.target import TargetModel, TargetConfig

    cfg = TargetConfig(num_layers=1, hidden=256, q_heads=2, kv_heads=1, head_dim=128, intermediate=512, vocab=5003)
    model = TargetModel.random(cfg, seed=5, dtype=torch.bfloat16, device=DEV)
    w = model.w["lm_head"]
    h = torch.randn(400, 256, device=DEV).to(torch.bfloat16)
    idx = torch.tensor(list(range(399, -1, -1)) + [7] * 37, dtype=torch.int32, device=DEV)  # 437 rows, repeats
    got = model.logits(h, row_index=idx)
    want = model.logits(h[idx.long()].contiguous())
    assert got.shape == (437, 5003) and torch.equal(got, want)
    assert rel_err(to_np(got), to_np(h[idx.long()].float() @ w.float().t())) < 2e-2
    out = torch.empty(437, 5003, dtype=torch.bfloat16, device=DEV)
    assert model.logits(h, row_index=idx, out=out).data_ptr() == out.data_ptr() and torch.equal(out, want)
    act = torch.ones(437, dtype=torch.int32, device=DEV)
    act[::3] = 0
    masked = torch.full((437, 5003), 9.0, dtype=torch.bfloat16, device=DEV)
    model.logits(h, row_index=idx, row_active=act, out=masked)
    on = act.bool()  # inactive rows may be left unwritten or written
    assert rel_err(to_np(masked[on]), to_np(want[on])) < 2e-2


def test_lm_head_topk_validates_out():
    """A caller's out tensor of the wrong shape, layout, dtype or alignment is refused
    before any launch."""
    x = torch.randn(8, 128, device=DEV).to(torch.bfloat16)
    w = torch.randn(1000, 128, device=DEV).to(torch.bfloat16)
    good = torch.empty(8, 1000, dtype=torch.bfloat16, device=DEV)
    ref = K().lm_head_topk(x, w, 0)[0]
    assert torch.equal(K().lm_head_topk(x, w, 0, out=good)[0], ref)
    bad = [torch.empty(7, 1000, dtype=torch.bfloat16, device=DEV),              # too few rows
           torch.empty(1000, 8, dtype=torch.bfloat16, device=DEV).t(),          # transposed
           torch.empty(8, 1004, dtype=torch.bfloat16, device=DEV)[:, 1:1001],   # stride 4k, base not 4-column aligned
           torch.empty(8, 1000, dtype=torch.float16, device=DEV)]               # dtype
    for o in bad:
        with pytest.raises((ValueError, TypeError)):
            K().lm_head_topk(x, w, 0, out=o)
    # a row stride that is not a multiple of 4 takes element stores: any base offset is fine
    odd = torch.empty(8, 1001, dtype=torch.bfloat16, device=DEV)[:, 1:]
    assert torch.equal(K().lm_head_topk(x, w, 0, out=odd)[0], ref)


def test_target_logits_topk_routes_and_matches():
    """TargetModel.logits_topk: the fused path (<= 256 bf16 rows) equals logits + top-k."""
    from flashgrpo_amd.models.target import TargetModel, TargetConfig

    cfg = TargetConfig(num_layers=1, hidden=128, q_heads=2, kv_heads=1, head_dim=64, intermediate=256, vocab=3001)
    model = TargetModel.random(cfg, seed=1, dtype=torch.bfloat16, device=DEV)
    h = torch.randn(150, 128, device=DEV).to(torch.bfloat16)
    lg, tok, sc, st = model.logits_topk(h, 5, stats=True, sanitize=True, logits=True)
    ref = model.logits(h)
    assert torch.equal(lg, ref)
    t2, s2, st2 = K().medusa_topk(ref, 5, stats=True, sanitize=True)
    assert torch.equal(tok, t2) and torch.equal(sc, s2)
    # 300 rows: the logits path (hipBLASLt) and the stand-alone top-k
    h3 = torch.randn(300, 128, device=DEV).to(torch.bfloat16)
    lg3, tok3, _, _ = model.logits_topk(h3, 3, logits=True)
    assert tok3.shape == (300, 3) and torch.equal(tok3, K().medusa_topk(lg3, 3)[0])


def _rank_keys_np(xs):
    """fg rank keys (value desc, index asc; NaN first, -0 == +0) of float32 rows, as uint64."""
    b = xs.astype(np.float32).view(np.uint32).astype(np.uint64)
    key = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    key = np.where(xs == 0, 0x80000000, key)
    key = np.where(np.isnan(xs), 0xFFFFFFFF, key).astype(np.uint64)
    idx = np.arange(xs.shape[-1], dtype=np.uint64)
    return (key << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)


@pytest.mark.parametrize("M,N,out_dtype", [(16, 152064, torch.bfloat16), (64, 32000, torch.bfloat16),
                                           (100, 5003, torch.float32), (200, 9000, torch.bfloat16)])
def test_row_maxima_parts(M, N, out_dtype):
    """The per-workgroup row maxima parts reduce to each row's maximum of the stored logits
    (NaN ignored) and to the rank key of its first maximum (NaN first)."""
    torch.manual_seed(M)
    Kd = 128
    src = (torch.randn(M + 5, Kd, device=DEV)).to(torch.bfloat16)
    w = (torch.randn(N, Kd, device=DEV) * 0.1).to(torch.bfloat16)
    w[N // 2] = w[N // 3]          # exact ties between two columns
    w[7, 0] = float("nan")         # a NaN column
    src[2, :] = 0.0                # a row of zeros: every logit is +-0 (and NaN in column 7)
    idx = torch.randperm(M + 5, device=DEV)[:M].to(torch.int32)
    P = K().lm_head_parts(N)
    pm = torch.empty(M, P, dtype=torch.float32, device=DEV)
    pk = torch.empty(M, P, dtype=torch.int64, device=DEV)
    lg = K().lm_head_topk(src, w, 0, row_index=idx, out_dtype=out_dtype, parts=(pm, pk))[0]
    ref = K().lm_head_topk(src, w, 0, row_index=idx, out_dtype=out_dtype)[0]
    xs = to_np(lg)
    assert np.array_equal(xs, to_np(ref), equal_nan=True)  # the parts do not change the logits
    want_max = np.where(np.isnan(xs), -np.inf, xs).max(axis=1)
    assert np.array_equal(to_np(pm).max(axis=1), want_max)
    keys = pk.cpu().numpy().view(np.uint64)
    assert np.array_equal(keys.max(axis=1), _rank_keys_np(xs).max(axis=1))


def test_row_maxima_parts_rejections():
    from flashgrpo_amd._lib import NativeError

    x = torch.randn(4, 64, device=DEV).to(torch.bfloat16)
    w = torch.randn(500, 64, device=DEV).to(torch.bfloat16)
    P = K().lm_head_parts(500)
    pm = torch.empty(4, P, dtype=torch.float32, device=DEV)
    pk = torch.empty(4, P, dtype=torch.int64, device=DEV)
    with pytest.raises((ValueError, NativeError)):
        K().lm_head_topk(x, w, 2, parts=(pm, pk))
    with pytest.raises(ValueError):
        K().lm_head_topk(x, w, 0, parts=(pm[:, :1].contiguous(), pk[:, :1].contiguous()))
