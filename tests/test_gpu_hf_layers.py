"""The decoder-layer kernels round where the reference's Hugging Face modules round.

The reference runs the Qwen2/Llama decoder layers of transformers under bf16 autocast
(flashgrpo/models/qwen_flashgrpo_wrapper.py:172-180). Its RMSNorm rounds x * rsqrt(mean x^2 + eps)
to bf16 before the weight product; its rotary embedding casts cos / sin to bf16 and rounds
q * cos, rotate_half(q) * sin and their sum; its MLP rounds SiLU(gate) before the product
with up. The installed transformers modules are run here on the same bf16 inputs and the
HIP kernels must agree bit for bit on all but a few elements (the mean of squares, cos / sin
and exp are evaluated by different code, so a rounding tie can fall either way). A kernel
that rounds once at the end agrees on far fewer elements (checked below by emulation).
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def K():
    from flashgrpo_amd import kernels

    return kernels


def frac_equal(a, b):
    return float((a.view(torch.int16) == b.view(torch.int16)).float().mean())


def test_rmsnorm_matches_qwen2_rmsnorm():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator(device=DEV).manual_seed(1)
    H = 3584
    x = (torch.randn(300, H, generator=g, device=DEV) * 3).to(BF)
    w = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).to(BF)
    norm = Qwen2RMSNorm(H, eps=1e-6).to(DEV, BF)
    with torch.no_grad():
        norm.weight.copy_(w)
        want = norm(x)
    got = K().rmsnorm(x.clone(), w, 1e-6)
    torch.cuda.synchronize()
    assert frac_equal(got, want) >= 0.999
    # rounding once at the end instead (the order the kernel had before) agrees far less often
    once = (x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()).to(BF)
    assert frac_equal(once, want) < 0.9


def test_rope_matches_qwen2_rotary_embedding():
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding, apply_rotary_pos_emb

    from flashgrpo_amd.models.target import inv_freq_table

    B, N, Hq, Hkv, d, S = 4, 29, 28, 4, 128, 2200
    cfg = Qwen2Config(hidden_size=Hq * d, num_attention_heads=Hq, num_key_value_heads=Hkv, rope_theta=1e6)
    rot = Qwen2RotaryEmbedding(config=cfg).to(DEV)
    assert torch.equal(inv_freq_table(d, 1e6).to(DEV), rot.inv_freq.float())
    g = torch.Generator(device=DEV).manual_seed(2)
    qkv = torch.randn(B * N, (Hq + 2 * Hkv) * d, generator=g, device=DEV).to(BF)
    seq = torch.tensor([0, 17, 900, 2047], dtype=torch.int32, device=DEV)
    pos_off = torch.randint(0, 5, (B, N), generator=g, device=DEV, dtype=torch.int32)
    qo = torch.empty(B, N, Hq, d, dtype=BF, device=DEV)
    kc = torch.zeros(B, Hkv, S, d, dtype=BF, device=DEV)
    vc = torch.zeros(B, Hkv, S, d, dtype=BF, device=DEV)
    K().rope_kv_write(qkv, batch=B, num_nodes=N, q_heads=Hq, kv_heads=Hkv, head_dim=d, seq_len=seq,
                      pos_offset=pos_off, inv_freq=inv_freq_table(d, 1e6).to(DEV), q_out=qo, k_cache=kc, v_cache=vc)
    x = qkv.view(B, N, Hq + 2 * Hkv, d)
    q, k = x[:, :, :Hq].transpose(1, 2), x[:, :, Hq:Hq + Hkv].transpose(1, 2)  # [B, heads, N, d]
    position_ids = (seq.view(B, 1) + pos_off).long()
    cos, sin = rot(x, position_ids)
    assert cos.dtype == BF
    qe, ke = apply_rotary_pos_emb(q, k, cos, sin)
    kgot = torch.stack([kc[b, :, int(seq[b]):int(seq[b]) + N] for b in range(B)])  # [B, Hkv, N, d]
    torch.cuda.synchronize()
    assert frac_equal(qo.transpose(1, 2), qe) >= 0.999
    assert frac_equal(kgot, ke) >= 0.999
    # fp32 cos / sin and one rounding at the end agree far less often
    c32, s32 = rot(x.float(), position_ids)
    c32, s32 = c32.unsqueeze(1), s32.unsqueeze(1)
    rh = torch.cat((-q.float()[..., d // 2:], q.float()[..., :d // 2]), dim=-1)
    once = (q.float() * c32 + rh * s32).to(BF)
    assert frac_equal(once, qe) < 0.97


def test_swiglu_matches_the_mlp_activation():
    g = torch.Generator(device=DEV).manual_seed(3)
    I = 18944
    gu = (torch.randn(200, 2 * I, generator=g, device=DEV) * 2).to(BF)
    want = F.silu(gu[:, :I]) * gu[:, I:]  # act_fn(gate_proj(x)) * up_proj(x) on bf16 tensors
    got = K().swiglu(gu)
    torch.cuda.synchronize()
    assert frac_equal(got, want) >= 0.999
    once = (F.silu(gu[:, :I].float()) * gu[:, I:].float()).to(BF)
    assert frac_equal(once, want) < 0.9
    # the flat grid reads rows of 2F and writes rows of F: other layouts are refused on the host
    with pytest.raises(ValueError):
        K().swiglu(gu[:, 8:8 + 2 * 96])  # a column slice (row stride 2I, not 2F)
    with pytest.raises(ValueError):
        K().swiglu(gu, out=torch.empty(200, 2 * I, dtype=BF, device=DEV)[:, :I])
    with pytest.raises(ValueError):
        K().swiglu(torch.zeros(4, 2 * 100, dtype=BF, device=DEV))  # F not a multiple of 8
    part = K().swiglu(gu[:64])  # a row slice is contiguous
    assert torch.equal(part, got[:64])


def test_medusa_block_matches_the_reference_head_under_autocast():
    """fg_medusa_heads against the reference's MedusaPredictionHead.project_hidden run the way its
    decoder runs it (flashgrpo/models/medusa_heads.py:74-78 under torch.autocast(bf16),
    flash_medusa_decoder.py:265-274): LayerNorm in fp32, fc in bf16, SiLU on the bf16 fc output,
    then the residual sum -- built here from torch.nn modules with fp32 master weights."""
    import torch.nn as nn

    torch.manual_seed(4)
    B, H = 64, 3584
    ln, fc = nn.LayerNorm(H).to(DEV), nn.Linear(H, H).to(DEV)
    with torch.no_grad():
        ln.weight.add_(torch.randn(H, device=DEV) * 0.1)
        ln.bias.add_(torch.randn(H, device=DEV) * 0.1)
        fc.weight.mul_(0.0).add_(torch.randn(H, H, device=DEV) * 0.02)
        fc.bias.add_(torch.randn(H, device=DEV) * 0.05)
    h = torch.randn(B, H, device=DEV).to(BF)
    with torch.no_grad(), torch.autocast("cuda", dtype=BF):
        want = h + F.silu(fc(ln(h)))
    assert want.dtype == BF
    got = K().medusa_heads(h, ln.weight.detach()[None], ln.bias.detach()[None],
                           fc.weight.detach().to(BF)[None].contiguous(), fc.bias.detach().to(BF)[None].contiguous(),
                           eps=ln.eps)
    torch.cuda.synchronize()
    # the fc sums run in a different order than the library GEMM, so a few roundings differ
    assert frac_equal(got, want) >= 0.98
    once_ref = (h.float() + F.silu(F.layer_norm(h.float(), (H,), ln.weight, ln.bias, ln.eps).to(BF).float()
                                   @ fc.weight.to(BF).float().t() + fc.bias.to(BF).float())).to(BF)
    assert frac_equal(once_ref, want) < 0.9
