"""The decoder projections as split-K GEMMs (``fg_linear_parts``) and the kernels that finish them
(``fg_residual_rmsnorm_parts``, ``fg_rope_kv_write_parts``).

* The parts, summed in split order, are checked against a float64 product within the fp32
  accumulation bound, over ragged rows/columns, padded row strides, every tile size and several
  split counts; with one split the four tile sizes accumulate each element in the same order and
  agree bit for bit (a transposed operand, a wrong column block or a dropped k-step fails the
  float64 check).
* The residual + RMSNorm kernel equals, bit for bit, the rounding chain of the Hugging Face
  decoder layer restated in torch (projection rounded to bf16, the residual sum rounded to bf16)
  followed by ``fg_rmsnorm`` (the same reduction order), and the norm stays within one bf16 step of
  a float64 RMSNorm.
* The rotary/cache-write kernel reading parts equals ``fg_rope_kv_write`` of the rows
  bf16(sum of parts + bias) bit for bit: the same q rows and the same cache slots, the rest of the
  cache untouched.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def K():
    from flashgrpo_amd import kernels

    return kernels


def operands(rows, hidden, cols, seed, *, x_pad=0, w_pad=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    xs = (torch.randn(rows, hidden + x_pad, device=DEV, generator=g) * 0.5).to(torch.bfloat16)
    ws = (torch.randn(cols, hidden + w_pad, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    return xs[:, :hidden], ws[:, :hidden]


def ordered_sum(parts):
    acc = parts[0].clone()
    for s in range(1, parts.shape[0]):
        acc += parts[s]
    return acc


def check_parts(parts, x, w):
    exact = x.double() @ w.double().t()
    S = parts.shape[0]
    Kd = x.shape[1]
    # fp32 accumulation of K/16 MFMA partial sums (each within 16 roundings) per split, plus the
    # S - 1 additions of the split sums
    bound = (Kd / 16 + 16 + S) * 2.0 ** -24 * (x.abs().double() @ w.abs().double().t()) + 1e-30
    err = (ordered_sum(parts).double() - exact).abs()
    assert bool((err <= bound).all()), f"worst excess {float((err - bound).max())}"


SHAPES = [(1, 64, 4), (37, 128, 200), (130, 192, 132), (257, 1536, 1000), (416, 1536, 2048)]


@pytest.mark.parametrize("rows,hidden,cols", SHAPES)
def test_parts_sum_matches_float64(rows, hidden, cols):
    x, w = operands(rows, hidden, cols, seed=rows + cols)
    ref = None
    for tile in ((64, 64), (64, 128), (128, 64), (128, 128)):
        for stages in (2, 3, 4):
            p = K().linear_parts(x, w, splits=1, tile=tile, stages=stages)
            check_parts(p, x, w)
            if ref is None:
                ref = p
            else:
                assert torch.equal(p, ref), f"tile {tile}, {stages} stages accumulate differently from (64, 64)"
    nk = hidden // 64
    for s in sorted({2, 3, 5, nk}):
        if s <= nk and K().linear_splits(hidden, s) == s:
            p = K().linear_parts(x, w, splits=s, tile=(128, 64))
            assert p.shape == (s, rows, cols)
            check_parts(p, x, w)
            assert torch.equal(p, K().linear_parts(x, w, splits=s, tile=(128, 64), stages=2))


def test_long_reduction_and_padded_strides():
    """The 1.5B down projection's reduction length (8960) with padded operand rows."""
    x, w = operands(96, 8960, 256, seed=5, x_pad=64, w_pad=8)
    for s in (1, 4, 7, 35, 70):  # 140 k-steps: from one split to two k-steps per split (fewer than the ring)
        s = K().linear_splits(8960, s)
        for stages in (2, 4):
            check_parts(K().linear_parts(x, w, splits=s, tile=(64, 128), stages=stages), x, w)


def test_invalid_split_counts_and_operands_are_rejected():
    x, w = operands(8, 192, 16, seed=1)
    assert K().linear_splits(192, 2) == 2 and K().linear_splits(1536, 7) == 6
    with pytest.raises(ValueError):
        K().linear_parts(x, w, splits=4)       # 3 k-steps
    with pytest.raises(ValueError):
        K().linear_parts(x, w, tile=(256, 64))
    with pytest.raises(ValueError):
        K().linear_parts(x, w, stages=5)
    with pytest.raises(ValueError):
        K().linear_parts(x[:, :100], w[:, :100])  # K not a multiple of 64
    with pytest.raises(ValueError):
        K().linear_parts(x, w[:14])            # N not a multiple of 4


@pytest.mark.parametrize("rows,H,S", [(1, 64, 1), (29, 1536, 3), (416, 1536, 5), (64, 3584, 2)])
def test_residual_rmsnorm_parts_follows_the_layer_rounding(rows, H, S):
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + H)
    parts = torch.randn(S, rows, H, device=DEV, generator=g) * 0.3
    x0 = (torch.randn(rows, H, device=DEV, generator=g)).to(torch.bfloat16)
    wt = (1.0 + 0.1 * torch.randn(H, device=DEV, generator=g)).to(torch.bfloat16)
    eps = 1e-6
    x = x0.clone()
    h = K().residual_rmsnorm_parts(parts, x, wt, eps)
    proj = ordered_sum(parts).to(torch.bfloat16)
    x_ref = (x0.float() + proj.float()).to(torch.bfloat16)
    assert torch.equal(x, x_ref)
    h_ref = K().rmsnorm(x_ref.clone(), wt, eps)
    assert torch.equal(h, h_ref)
    # against a float64 RMSNorm: x * rsqrt(mean x^2 + eps) rounded to bf16, then times the weight
    xd = x_ref.double()
    n = (xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16).double()
    h64 = (wt.double() * n).to(torch.bfloat16).double()
    assert bool(((h.double() - h64).abs() <= 2.0 ** -6 * h64.abs() + 1e-30).all())


@pytest.mark.parametrize("with_bias,per_seq_pos", [(True, False), (False, True)])
def test_rope_kv_write_parts_equals_rope_of_rounded_rows(with_bias, per_seq_pos):
    B, N, Hq, Hkv, d, cap = 3, 13, 12, 2, 128, 64
    width = (Hq + 2 * Hkv) * d
    g = torch.Generator(device=DEV).manual_seed(11 + with_bias)
    S = 3
    parts = torch.randn(S, B * N, width, device=DEV, generator=g)
    bias = (0.1 * torch.randn(width, device=DEV, generator=g)).to(torch.bfloat16) if with_bias else None
    seq_len = torch.tensor([5, 17, 30], dtype=torch.int32, device=DEV)
    if per_seq_pos:
        pos = torch.randint(0, 4, (B, N), dtype=torch.int32, device=DEV, generator=g)
    else:
        pos = torch.arange(N, dtype=torch.int32, device=DEV) // 3
    inv_freq = 1.0 / (1.0e6 ** (torch.arange(0, d, 2, device=DEV).float() / d))
    cache0 = torch.randn(B, Hkv, cap, d, device=DEV, generator=g).to(torch.bfloat16)
    kc, vc, q = cache0.clone(), cache0.clone(), torch.empty(B, N, Hq, d, dtype=torch.bfloat16, device=DEV)
    K().rope_kv_write_parts(parts, bias, batch=B, num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=d, seq_len=seq_len,
                            pos_offset=pos, inv_freq=inv_freq, q_out=q, k_cache=kc, v_cache=vc)
    rows = ordered_sum(parts) + (bias.float() if with_bias else 0.0)
    qkv = rows.to(torch.bfloat16)
    kr, vr, qr = cache0.clone(), cache0.clone(), torch.empty_like(q)
    K().rope_kv_write(qkv, batch=B, num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=d, seq_len=seq_len,
                      pos_offset=pos, inv_freq=inv_freq, q_out=qr, k_cache=kr, v_cache=vr)
    torch.cuda.synchronize()
    assert torch.equal(q, qr)
    assert torch.equal(kc, kr)
    assert torch.equal(vc, vr)
    assert not torch.equal(kc, cache0)  # the tree slots were written


@pytest.mark.parametrize("tile,stages", [((64, 64), 4), ((64, 128), 2), ((128, 64), 3), ((128, 128), 4),
                                         ((128, 128), 2)])
@pytest.mark.parametrize("with_bias,per_seq_pos,mapped", [(True, False, False), (False, True, True)])
def test_linear_rope_kv_write_equals_parts_then_rope(tile, stages, with_bias, per_seq_pos, mapped):
    """The q/k/v projection with the bias, rotary embedding and KV-slot write in its epilogue
    (pair-interleaved weight rows) writes exactly what fg_linear_parts (one split, the same tile and
    ring) followed by fg_rope_kv_write_parts writes: the same q rows and cache slots, the rest of the
    cache untouched. Ragged row counts, per-sequence position offsets and a row map included."""
    B, N, Hq, Hkv, d, cap, Kd = 5, 13, 12, 2, 128, 64, 384
    width = (Hq + 2 * Hkv) * d
    x, w = operands(B * N, Kd, width, seed=21 + stages)
    g = torch.Generator(device=DEV).manual_seed(3)
    bias = (0.1 * torch.randn(width, device=DEV, generator=g)).to(torch.bfloat16) if with_bias else None
    seq_len = torch.tensor([5, 17, 30, 0, 40], dtype=torch.int32, device=DEV)
    if per_seq_pos:
        pos = torch.randint(0, 4, (B, N), dtype=torch.int32, device=DEV, generator=g)
    else:
        pos = torch.arange(N, dtype=torch.int32, device=DEV) // 3
    row_map = torch.tensor([4, 2, 0, 1, 3], dtype=torch.int32, device=DEV) if mapped else None
    inv_freq = 1.0 / (1.0e6 ** (torch.arange(0, d, 2, device=DEV).float() / d))
    cache0 = torch.randn(B, Hkv, cap, d, device=DEV, generator=g).to(torch.bfloat16)
    rope = dict(batch=B, num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=d, seq_len=seq_len, pos_offset=pos,
                inv_freq=inv_freq, row_map=row_map)
    kr, vr, qr = cache0.clone(), cache0.clone(), torch.empty(B, N, Hq, d, dtype=torch.bfloat16, device=DEV)
    parts = K().linear_parts(x, w, splits=1, tile=tile, stages=stages)
    K().rope_kv_write_parts(parts, bias, q_out=qr, k_cache=kr, v_cache=vr, **rope)
    wp = K().rope_pair_rows(w, Hq, Hkv, d)
    bp = None if bias is None else K().rope_pair_rows(bias, Hq, Hkv, d)
    kc, vc, q = cache0.clone(), cache0.clone(), torch.empty_like(qr)
    K().linear_rope_kv_write(x, wp, bp, tile=tile, stages=stages, q_out=q, k_cache=kc, v_cache=vc, **rope)
    torch.cuda.synchronize()
    assert torch.equal(q, qr)
    assert torch.equal(kc, kr)
    assert torch.equal(vc, vr)
    assert not torch.equal(kc, cache0)


def test_linear_rope_kv_write_flags_slots_outside_the_cache():
    """A row whose cache slot falls outside the cache is not written and sets bit 8 of the error
    flag, as fg_rope_kv_write_parts does; its q row is still written."""
    B, N, Hq, Hkv, d, cap, Kd = 2, 4, 4, 1, 64, 8, 128
    width = (Hq + 2 * Hkv) * d
    x, w = operands(B * N, Kd, width, seed=4)
    seq_len = torch.tensor([2, 6], dtype=torch.int32, device=DEV)  # sequence 1's slots 6..9 reach past 8
    pos = torch.arange(N, dtype=torch.int32, device=DEV)
    inv_freq = 1.0 / (1.0e6 ** (torch.arange(0, d, 2, device=DEV).float() / d))
    outs = []
    for fused in (False, True):
        kc = torch.zeros(B, Hkv, cap, d, dtype=torch.bfloat16, device=DEV)
        vc, q = torch.zeros_like(kc), torch.zeros(B, N, Hq, d, dtype=torch.bfloat16, device=DEV)
        flag = torch.zeros(1, dtype=torch.int32, device=DEV)
        rope = dict(batch=B, num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=d, seq_len=seq_len, pos_offset=pos,
                    inv_freq=inv_freq, q_out=q, k_cache=kc, v_cache=vc, err_flag=flag)
        if fused:
            K().linear_rope_kv_write(x, K().rope_pair_rows(w, Hq, Hkv, d), None, **rope)
        else:
            K().rope_kv_write_parts(K().linear_parts(x, w, splits=1, tile=(64, 64)), None, **rope)
        torch.cuda.synchronize()
        outs.append((q, kc, vc, int(flag.item())))
    assert outs[0][3] == outs[1][3] == 8
    for a, b in zip(outs[0][:3], outs[1][:3]):
        assert torch.equal(a, b)
