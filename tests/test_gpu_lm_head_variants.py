"""Every instantiation of the weight-streaming LM head that ``fg_lm_head_topk`` can
reach, one parity case each.

The kernel template is instantiated per row-block count (1-64, 65-128, 129-192 and
193-256 rows), output dtype (bf16, fp32), top-k bucket (none, 1, 2, 4, 8, 16; 16 only up
to 192 rows), sanitising and row-maxima parts; each instantiation compiles to its own
register allocation around the inline-asm weight loads, so each gets a case here. The
logits are checked against an fp32 product, the candidates and (max, logsumexp) against
``oracle.tree.topk_canonical`` on the kernel's own bf16 logits, the parts against the
row maxima of the stored logits. The Medusa fc instantiations (1-64, 65-128, 129-256
rows) are covered by ``test_gpu_kernels.py::test_medusa_heads_stream_matches_fp32_reference``.
"""
import numpy as np
import pytest
import torch

from oracle import tree as OT

pytestmark = pytest.mark.gpu
DEV = "cuda"
ROWS = [40, 100, 170, 230]      # 2, 4, 6 and 8 row blocks of 32
KMAX = [1, 2, 3, 5, 12]         # buckets 1, 2, 4, 8, 16


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def K():
    from flashgrpo_amd import kernels

    return kernels


def to_np(t):
    return t.detach().float().cpu().numpy()


def rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _rank_keys_np(xs):
    b = xs.astype(np.float32).view(np.uint32).astype(np.uint64)
    key = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    key = np.where(xs == 0, 0x80000000, key)
    key = np.where(np.isnan(xs), 0xFFFFFFFF, key).astype(np.uint64)
    idx = np.arange(xs.shape[-1], dtype=np.uint64)
    return (key << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)


@pytest.mark.parametrize("M", ROWS)
def test_every_reachable_instantiation(M):
    g = torch.Generator(device="cpu").manual_seed(M)
    N, Kd = 4099, 192  # a partial last column block
    x = torch.randn(M + 7, Kd, generator=g)
    x[: M // 4] = torch.randint(-3, 4, (M // 4, Kd), generator=g).float()  # rows with tied logits
    w = torch.randint(-2, 3, (N, Kd), generator=g).float() * 0.125
    w[N // 2:] = torch.randn(N - N // 2, Kd, generator=g) * 0.05
    xd, wd = x.to(torch.bfloat16).to(DEV), w.to(torch.bfloat16).to(DEV)
    idx = torch.randperm(M + 7, generator=g)[:M].to(torch.int32).to(DEV)
    rows = xd[idx.long()].contiguous()
    ref32 = to_np(rows.float() @ wd.float().t())

    # logits only, both output dtypes, contiguous and gathered rows
    base = K().lm_head_topk(rows, wd, 0)[0]
    assert rel_err(to_np(base), ref32) < 2e-2
    base32 = K().lm_head_topk(rows, wd, 0, out_dtype=torch.float32)[0]
    assert rel_err(to_np(base32), ref32) < 1e-5
    assert torch.equal(K().lm_head_topk(xd, wd, 0, row_index=idx)[0], base)
    assert torch.equal(base32.to(torch.bfloat16), base)

    # row-maxima parts with both output dtypes
    P = K().lm_head_parts(N)
    for od, lg_ref in ((torch.bfloat16, base), (torch.float32, base32)):
        pm = torch.empty(M, P, dtype=torch.float32, device=DEV)
        pk = torch.empty(M, P, dtype=torch.int64, device=DEV)
        lg = K().lm_head_topk(xd, wd, 0, row_index=idx, out_dtype=od, parts=(pm, pk))[0]
        assert torch.equal(lg, lg_ref), od
        xs = to_np(lg)
        assert np.array_equal(to_np(pm).max(axis=1), xs.max(axis=1)), od
        assert np.array_equal(pk.cpu().numpy().view(np.uint64).max(axis=1), _rank_keys_np(xs).max(axis=1)), od

    # top-k buckets x sanitising x (no logits, bf16 logits, fp32 logits); the candidates rank
    # the bf16-rounded values in every case
    xs = to_np(base)
    want = {}
    for san in (False, True):
        tops = [OT.topk_canonical(OT.nan_to_num_logits(r) if san else r, 16) for r in xs]
        want[san] = (np.stack([t[0] for t in tops]), np.stack([t[1] for t in tops]).astype(np.float32) + 0.0)
    m = xs.max(axis=1)
    lse = np.log(np.exp(xs.astype(np.float64) - m[:, None]).sum(axis=1)) + m
    for kmax in KMAX:
        if kmax > 8 and M > 192:
            with pytest.raises(Exception, match="kmax above 8"):
                K().lm_head_topk(rows, wd, kmax)
            continue
        for san in (False, True):
            for mode in (None, torch.bfloat16, torch.float32):
                lg, tok, sc, st = K().lm_head_topk(rows, wd, kmax, logits=mode is not None, out_dtype=mode,
                                                   stats=True, sanitize=san)
                case = (kmax, san, mode)
                assert np.array_equal(tok.cpu().numpy(), want[san][0][:, :kmax]), case
                assert np.array_equal(to_np(sc), want[san][1][:, :kmax]), case
                assert np.array_equal(to_np(st[:, 0]), m), case
                assert np.max(np.abs(to_np(st[:, 1]) - lse) / np.maximum(1.0, np.abs(lse))) < 1e-4, case
                if mode is None:
                    assert lg is None
                else:
                    assert torch.equal(lg, base if mode == torch.bfloat16 else base32), case
