"""The fused MLP input GEMM ``fg_gate_up_swiglu``: SiLU(bf16(x.Wg^T)) * bf16(x.Wu^T) in one kernel.

Checked against a float64 product rounded the way the unfused path and the reference's MLP
under bf16 autocast round (gate and up to bf16, SiLU(gate) to bf16, the product to bf16): every element within the error that one bf16
rounding flip of gate or up can cause, and almost every element bit-equal (a dropped rounding,
a swapped gate/up block or a wrong column block fails the second check). The kernel is also
compared with the unfused pair it replaces (hipBLASLt projection + ``fg_swiglu``), with both tile
heights (which accumulate every element in the same order, so agree bit for bit), over ragged
row and column counts, strided operands and output padding that must stay untouched.
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def K():
    from flashgrpo_amd import kernels

    return kernels


def operands(rows, hidden, inter, seed, *, x_pad=0, w_pad=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    xs = (torch.randn(rows, hidden + x_pad, device=DEV, generator=g) * 0.5).to(torch.bfloat16)
    ws = (torch.randn(2 * inter, hidden + w_pad, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    return xs[:, :hidden], ws[:, :hidden]


def reference(x, w):
    """float64 products -> bf16 gate/up -> bf16 SiLU(gate) -> times up in fp32 -> bf16 (the rounding
    points of the Hugging Face MLP under bf16 autocast), and the bf16 gate/up."""
    inter = w.shape[0] // 2
    gu = (x.double() @ w.double().t()).float().to(torch.bfloat16)
    gt, up = gu[:, :inter].float(), gu[:, inter:].float()
    act = (gt / (1.0 + torch.exp(-gt))).to(torch.bfloat16).float()
    return (act * up).to(torch.bfloat16), gt, up


def accumulation_error(x, w):
    """Bound on |fp32 sum - exact sum| of each gate/up product: (K/16 + 16) * 2^-24 * sum_k |x_k w_k|
    (K/16 fp32 accumulations of 16-product MFMA partial sums, each partial sum within 16 roundings)."""
    K = x.shape[1]
    return (K / 16 + 16) * 2.0 ** -24 * (x.abs().double() @ w.abs().double().t()).float()


def check_against_reference(out, x, w, min_exact=0.99):
    ref, gt, up = reference(x, w)
    o, r = out.float(), ref.float()
    inter = w.shape[0] // 2
    err = accumulation_error(x, w)
    eg, eu = err[:, :inter], err[:, inter:]
    # gate and up may each differ from the rounded exact products by their fp32 accumulation error
    # plus one bf16 rounding flip (2^-7 of the value), and the bf16 SiLU(gate) by one more flip;
    # SiLU' <= 1.1 and |SiLU(g)| <= |g|, so SiLU(gate)*up moves by
    # <= (1.1 (2^-7 |g| + eg) + 2^-7 |g|) (|u| + eu) + (|g| + eg) (2^-7 |u| + eu);
    # the result's own rounding may then differ by one ulp (2^-7 |o|)
    ag, au = gt.abs(), up.abs()
    tol = ((1.1 * (2.0 ** -7 * ag + eg) + 2.0 ** -7 * ag) * (au + eu) + (ag + eg) * (2.0 ** -7 * au + eu)
           + 2.0 ** -6 * r.abs() + 1e-30)
    bad = (o - r).abs() > tol
    assert not bad.any(), f"{int(bad.sum())} elements outside the one-flip bound; worst {float((o - r).abs().max())}"
    exact = float((out.view(torch.int16) == ref.view(torch.int16)).float().mean())
    assert exact >= min_exact, f"only {exact:.4%} of elements bit-equal to the rounded float64 reference"
    return exact


@pytest.mark.parametrize("rows,hidden,inter", [(1, 64, 4), (37, 128, 200), (193, 192, 132), (257, 1536, 1000),
                                               (385, 256, 8960 // 8)])
def test_matches_rounded_float64_reference(rows, hidden, inter):
    x, w = operands(rows, hidden, inter, seed=rows + inter)
    out = K().gate_up_swiglu(x, w)
    torch.cuda.synchronize()
    check_against_reference(out, x, w)


@pytest.mark.parametrize("tile_rows", [64, 128, 192, 256])
def test_every_tile_height_agrees_bitwise(tile_rows):
    x, w = operands(300, 512, 520, seed=5)
    auto = K().gate_up_swiglu(x, w)
    forced = K().gate_up_swiglu(x, w, tile_rows=tile_rows)
    torch.cuda.synchronize()
    assert torch.equal(auto.view(torch.int16), forced.view(torch.int16))
    check_against_reference(forced, x, w)


def test_strided_operands_and_untouched_padding():
    rows, hidden, inter = 211, 320, 260
    x, w = operands(rows, hidden, inter, seed=11, x_pad=64, w_pad=128)
    assert x.stride(0) == hidden + 64 and w.stride(0) == hidden + 128
    big = torch.full((rows, inter + 12), -7.0, dtype=torch.bfloat16, device=DEV)
    out = big[:, :inter]
    K().gate_up_swiglu(x, w, out=out)
    torch.cuda.synchronize()
    assert torch.equal(big[:, inter:], torch.full_like(big[:, inter:], -7.0))
    check_against_reference(out, x, w)
    dense = K().gate_up_swiglu(x.contiguous(), w.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(dense.view(torch.int16), out.contiguous().view(torch.int16))


@pytest.mark.parametrize("rows,hidden,inter,tile", [(1856, 3584, 18944, 0), (512, 1536, 8960, 0),
                                                    (416, 1536, 8960, 64), (416, 1536, 8960, 128)])
def test_decoder_shapes_match_the_unfused_pair(rows, hidden, inter, tile):
    """Qwen2.5-7B and 1.5B verify-round shapes (B x tree nodes rows) against the projection +
    SwiGLU kernels it replaces, and against the rounded float64 reference."""
    x, w = operands(rows, hidden, inter, seed=rows)
    fused = K().gate_up_swiglu(x, w, tile_rows=tile)
    unfused = K().swiglu(F.linear(x, w))
    torch.cuda.synchronize()
    same = float((fused.view(torch.int16) == unfused.view(torch.int16)).float().mean())
    assert same >= 0.999, f"{same:.5%} bit-equal to hipBLASLt + fg_swiglu"
    check_against_reference(fused, x, w, min_exact=0.999)


def test_rejects_unsupported_operands():
    x, w = operands(8, 64, 8, seed=1)
    with pytest.raises(ValueError):
        K().gate_up_swiglu(x.float(), w.float())
    x2, w2 = operands(8, 96, 8, seed=1)  # hidden not a multiple of 64
    with pytest.raises(ValueError):
        K().gate_up_swiglu(x2, w2)
    with pytest.raises(ValueError):
        K().gate_up_swiglu(x, w, out=torch.empty(8, 9, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError, match="tile_rows"):
        K().gate_up_swiglu(x, w, tile_rows=96)
