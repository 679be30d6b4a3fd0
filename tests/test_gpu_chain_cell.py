"""The ChainDraftCell's input normalisation on the device (``fg_chain_cell_norm``) and the cell step.

Checked against a float64 LayerNorm of the same inputs (mean, then mean squared deviation;
the affine weights as the device holds them): every element within one rounding of the
output dtype plus an fp32 accumulation bound, and in bf16 almost every element bit-equal to
the rounded float64 value (a dropped bias, a swapped weight pair or a variance without the
mean fail those checks), and the cell step against the module's own torch forward.
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


def ln64(x, w, b, eps):
    x = x.double()
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + eps) * w.double() + b.double()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,H,pad", [(1, 8, 0), (7, 1000, 8), (300, 4096, 0), (33, 8192, 16)])
def test_matches_float64_layer_norms(dtype, rows, H, pad):
    g = torch.Generator(device=DEV).manual_seed(rows * H)
    st = (torch.randn(rows, H + pad, generator=g, device=DEV) * 3 + 1).to(dtype)[:, :H]
    tk = (torch.randn(rows, H + pad, generator=g, device=DEV) * 0.2 - 0.5).to(dtype)[:, :H]
    sw, sb, tw, tb = [(torch.randn(H, generator=g, device=DEV) * s + o).to(dtype)
                      for s, o in ((0.1, 1.0), (0.1, 0.0), (0.2, 1.0), (0.05, 0.1))]
    eps = 1e-5
    out = K().chain_cell_norm(st, tk, sw, sb, tw, tb, eps)
    torch.cuda.synchronize()
    ref = torch.cat([ln64(st, sw, sb, eps), ln64(tk, tw, tb, eps)], dim=-1)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -22
    # output rounding (one ulp of the value) + fp32 statistics: |x - mean| * rstd relative 2^-20,
    # times |w|, plus the same for the bias-free part
    w2 = torch.cat([sw, tw]).double().abs()
    tol = ulp * ref.abs() + 2.0 ** -18 * (ref.abs() + w2 * 8) + 1e-30
    err = (out.double() - ref).abs()
    assert (err <= tol).all(), f"worst {float((err - tol).max())}"
    if dtype == torch.bfloat16:
        exact = float((out == ref.to(dtype)).float().mean())
        assert exact >= 0.99, exact
    torch_ref = torch.cat([F.layer_norm(st, (H,), sw, sb, eps), F.layer_norm(tk, (H,), tw, tb, eps)], dim=-1)
    assert float((out.float() - torch_ref.float()).abs().max()) <= 2 * ulp * float(torch_ref.float().abs().max())


@pytest.mark.parametrize("cell_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("state_dtype", [torch.bfloat16, torch.float32])
def test_cell_step_matches_module_forward(cell_dtype, state_dtype):
    """The step runs in the cell's parameter dtype, whatever the state's (the rollout hands
    it bf16 hidden rows and fp32 states of fp32 heads), and returns that dtype, as the
    module's forward does. In fp32 it agrees with the forward to fp32 rounding; in bf16
    almost every element is bit-equal (only the LayerNorm, one HIP launch, differs from
    torch's, by a bf16 rounding flip now and then)."""
    from flashgrpo_amd.models.medusa_heads import ChainDraftCell

    torch.manual_seed(3)
    H = 512
    cell = ChainDraftCell(H, gate_init=-1.0).to(DEV)
    with torch.no_grad():
        for p in cell.parameters():
            p.add_(torch.randn_like(p) * 0.05)
    cell = cell.to(cell_dtype)
    state = (torch.randn(37, H, device=DEV) * 2).to(state_dtype)
    tok = torch.randn(37, H, device=DEV).to(torch.bfloat16)
    got = cell.step(state, tok)
    with torch.no_grad():
        want = cell(state, tok)
    torch.cuda.synchronize()
    assert got.dtype == want.dtype == cell_dtype
    if cell_dtype == torch.float32:
        assert float((got - want).abs().max()) <= 1e-5 * float(want.abs().max())
    else:
        exact = float((got.view(torch.int16) == want.view(torch.int16)).float().mean())
        assert exact >= 0.97, exact
        assert float((got.float() - want.float()).abs().max()) <= 2.0 ** -6 * float(want.float().abs().max())


def test_chain_bootstrap_head_runs_in_its_parameter_dtype():
    """Medusa head 0 bootstraps chain proposals outside autocast: fp32 heads give an fp32
    state from the bf16 hidden rows, h + SiLU(fc(LayerNorm(h))) with no bf16 rounding."""
    from flashgrpo_amd.models.medusa_heads import MedusaHeads

    torch.manual_seed(5)
    H = 512
    heads = MedusaHeads(H, 1000, 2).to(DEV)
    with torch.no_grad():
        for p in heads.parameters():
            p.add_(torch.randn_like(p) * 0.05)
    hid = (torch.randn(21, H, device=DEV) * 2).to(torch.bfloat16)
    got = heads.heads[0].project_hidden(hid)
    hd = heads.heads[0]
    with torch.no_grad():
        x = hid.double()
        want = x + F.silu(F.linear(F.layer_norm(x, (H,), hd.norm.weight.double(), hd.norm.bias.double(), hd.norm.eps),
                                   hd.fc.weight.double(), hd.fc.bias.double()))
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    assert float((got.double() - want).abs().max()) <= 1e-5 * float(want.abs().max())


def test_rejects_bad_operands():
    x = torch.zeros(4, 12, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(12, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="multiple of 8"):
        K().chain_cell_norm(x, x, w, w, w, w, 1e-5)
    x = torch.zeros(4, 16, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        K().chain_cell_norm(x, x.float(), w, w, w, w, 1e-5)
