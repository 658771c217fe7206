"""K6 (sf_rms_norm) against transformers' Qwen3MoeRMSNorm and a float64
evaluation of the same formula (tf:294-299).  The kernel sums the squares
in its own fp32 order, so its output may differ from the eager module's by
the rounding of the variance.  That moves the first bf16 rounding by at
most one step, which the weight multiply and the second rounding can turn
into two: the tests bound the difference to two bf16 steps and require
nearly every element to be bitwise equal."""
import math

import pytest
import torch

from specfit_amd import ops
from specfit_amd.runtime import Qwen3RMSNormHip, install_hip_norms

pytestmark = pytest.mark.gpu


def _bf16_steps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in units of the bf16 spacing at b (elementwise)."""
    a, b = a.float(), b.float()
    exp = torch.floor(torch.log2(b.abs().clamp_min(2.0 ** -126)))
    return (a - b).abs() / torch.exp2(exp - 7)


def _reference_f64(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """The eager formula with the variance in float64, then the module's two
    bf16 rounding points."""
    xf = x.double()
    var = xf.pow(2).mean(-1, keepdim=True)
    y = (xf * torch.rsqrt(var + eps)).to(torch.bfloat16)
    return (w.double() * y.double()).to(torch.bfloat16)


@pytest.mark.parametrize("shape", [(61, 2048), (1, 61, 32, 128), (1, 61, 4, 128), (3, 4096),
                                   (7, 24), (5, 40), (2, 8, 13)])
def test_rms_norm_matches_the_eager_module(device, shape):
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeRMSNorm

    torch.manual_seed(sum(shape))
    dim = shape[-1]
    x = (torch.randn(shape, device=device) * 3).to(torch.bfloat16)
    eager = Qwen3MoeRMSNorm(dim, eps=1e-6).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        eager.weight.copy_((1 + 0.1 * torch.randn(dim, device=device)).to(torch.bfloat16))
    hip = Qwen3RMSNormHip.from_module(eager)
    with torch.no_grad():
        expected = eager(x)
        actual = hip(x)
    torch.cuda.synchronize()
    assert actual.shape == expected.shape and actual.dtype == torch.bfloat16
    steps = _bf16_steps(actual, expected)
    exact = (actual == expected).float().mean().item()
    print(f"{shape}: {exact:.4%} bitwise equal to the eager module, "
          f"max {steps.max().item():.0f} bf16 steps", flush=True)
    assert steps.max().item() <= 2.0, shape
    assert exact >= 0.98
    ref = _reference_f64(x, eager.weight, 1e-6)
    assert _bf16_steps(actual, ref).max().item() <= 2.0


def test_rms_norm_of_strided_views_and_empty_inputs(device):
    torch.manual_seed(3)
    w = torch.randn(128, device=device).to(torch.bfloat16)
    base = torch.randn(61, 4096, device=device).to(torch.bfloat16)
    view = base.view(1, 61, 32, 128)
    assert torch.equal(ops.rms_norm(view, w, 1e-6), ops.rms_norm(view.contiguous(), w, 1e-6))
    # rows at a non-contiguous stride: every other row of the matrix
    rows = base[::2, :128]
    assert torch.equal(ops.rms_norm(rows, w, 1e-6), ops.rms_norm(rows.contiguous(), w, 1e-6))
    empty = torch.empty(0, 128, dtype=torch.bfloat16, device=device)
    assert ops.rms_norm(empty, w, 1e-6).shape == (0, 128)
    with pytest.raises(ValueError):
        ops.rms_norm(base, w, 1e-6)  # weight of the wrong length


def test_installing_hip_norms_keeps_the_model_output(device):
    """The Qwen3-MoE dense path with its norms on K6 stays within bf16
    rounding of the eager norms (experts replaced by identity to isolate
    the norms)."""
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    torch.manual_seed(7)
    cfg = Qwen3MoeConfig(vocab_size=128, hidden_size=256, intermediate_size=256,
                         moe_intermediate_size=64, num_hidden_layers=2, num_attention_heads=4,
                         num_key_value_heads=2, head_dim=64, num_experts=4,
                         num_experts_per_tok=2, max_position_embeddings=64)
    model = Qwen3MoeForCausalLM(cfg).to(device=device, dtype=torch.bfloat16).eval()
    ids = torch.randint(0, 128, (1, 12), device=device)
    with torch.no_grad():
        expected = model(ids).logits.float()
        replaced = install_hip_norms(model)
        actual = model(ids).logits.float()
    assert replaced == 2 * 4 + 1  # four per decoder layer and the final norm
    assert isinstance(model.model.norm, Qwen3RMSNormHip)
    err = (actual - expected).abs().max().item() / expected.abs().max().item()
    assert err < 2e-2, err
    assert not math.isnan(err)


def _attention_config(head_dim):
    from transformers import Qwen3MoeConfig

    return Qwen3MoeConfig(vocab_size=128, hidden_size=256, intermediate_size=256,
                          moe_intermediate_size=64, num_hidden_layers=1, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=head_dim, num_experts=4,
                          num_experts_per_tok=2, max_position_embeddings=256,
                          attn_implementation="sdpa")


@pytest.mark.parametrize("tokens", [1, 7, 61, 128])
def test_qk_norm_rope_equals_the_eager_sequence_bitwise(device, tokens):
    """K7 against the eager sequence of Qwen3MoeAttention.forward (tf:162-167)
    with the norms on K6: q_norm/k_norm, transpose, apply_rotary_pos_emb."""
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (Qwen3MoeRotaryEmbedding,
                                                                    apply_rotary_pos_emb)

    torch.manual_seed(tokens)
    Hq, Hk, D = 32, 4, 128
    q = (torch.randn(1, tokens, Hq, D, device=device) * 2).to(torch.bfloat16)
    k = (torch.randn(1, tokens, Hk, D, device=device) * 2).to(torch.bfloat16)
    wq = (1 + 0.2 * torch.randn(D, device=device)).to(torch.bfloat16)
    wk = (1 + 0.2 * torch.randn(D, device=device)).to(torch.bfloat16)
    cfg = _attention_config(D)
    rope = Qwen3MoeRotaryEmbedding(cfg).to(device)
    positions = (1000 + torch.arange(tokens, device=device)).unsqueeze(0)
    cos, sin = rope(q, positions)
    qn = Qwen3RMSNormHip(torch.nn.Parameter(wq), 1e-6)
    kn = Qwen3RMSNormHip(torch.nn.Parameter(wk), 1e-6)
    eq, ek = apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
    aq, ak = ops.qk_norm_rope(q, k, wq, wk, 1e-6, cos, sin)
    assert aq.shape == (1, Hq, tokens, D) and ak.shape == (1, Hk, tokens, D)
    assert torch.equal(aq, eq) and torch.equal(ak, ek)


@pytest.mark.parametrize("tokens", [1, 5, 64])
def test_qk_norm_rope_reads_heads_out_of_fused_projection_rows(device, tokens):
    """q and k as views into one [tokens, (Hq + 2 Hk) * 128] projection
    output (token stride 5120 elements, like Qwen3-30B-A3B's fused q/k/v
    rows) give the bits of the same heads copied out contiguously."""
    torch.manual_seed(100 + tokens)
    Hq, Hk, D = 32, 4, 128
    rows = (torch.randn(1, tokens, (Hq + 2 * Hk) * D, device=device) * 2).to(torch.bfloat16)
    q = rows[..., :Hq * D].view(1, tokens, Hq, D)
    k = rows[..., Hq * D:(Hq + Hk) * D].view(1, tokens, Hk, D)
    assert not q.is_contiguous() or tokens == 1
    wq = (1 + 0.2 * torch.randn(D, device=device)).to(torch.bfloat16)
    wk = (1 + 0.2 * torch.randn(D, device=device)).to(torch.bfloat16)
    ang = torch.rand(1, tokens, D, device=device) * 6.2
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    aq, ak = ops.qk_norm_rope(q, k, wq, wk, 1e-6, cos, sin)
    eq, ek = ops.qk_norm_rope(q.contiguous(), k.contiguous(), wq, wk, 1e-6, cos, sin)
    assert torch.equal(aq, eq) and torch.equal(ak, ek)


def test_qk_norm_rope_rejects_unaligned_token_strides(device):
    rows = torch.zeros(1, 3, 4 * 128 + 4, dtype=torch.bfloat16, device=device)
    q = rows[..., :4 * 128].view(1, 3, 4, 128)
    w = torch.ones(128, dtype=torch.bfloat16, device=device)
    cs = torch.zeros(1, 3, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="multiple of 8"):
        ops.qk_norm_rope(q, q, w, w, 1e-6, cs, cs)


@pytest.mark.parametrize("head_dim", [128, 64])
def test_hip_attention_module_matches_the_hf_module(device, head_dim):
    """Qwen3AttentionHip (fused at head_dim 128, eager norms+rotary at 64)
    gives the HF module's output bit for bit when both use K6 norms."""
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (Qwen3MoeAttention,
                                                                    Qwen3MoeRotaryEmbedding)

    from specfit_amd.runtime import Qwen3AttentionHip

    torch.manual_seed(head_dim)
    cfg = _attention_config(head_dim)
    hf = Qwen3MoeAttention(cfg, layer_idx=0).to(device=device, dtype=torch.bfloat16).eval()
    with torch.no_grad():
        for norm in (hf.q_norm, hf.k_norm):
            norm.weight.copy_((1 + 0.2 * torch.randn(head_dim, device=device)).to(torch.bfloat16))
    hf.q_norm = Qwen3RMSNormHip.from_module(hf.q_norm)
    hf.k_norm = Qwen3RMSNormHip.from_module(hf.k_norm)
    hip = Qwen3AttentionHip.from_module(hf)
    T = 12
    h = torch.randn(1, T, 256, device=device).to(torch.bfloat16)
    pos = torch.arange(T, device=device).unsqueeze(0)
    emb = Qwen3MoeRotaryEmbedding(cfg).to(device)(h, pos)
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool, device=device)).view(1, 1, T, T)
    assert hip._fused_projection()
    with torch.no_grad():
        expected, _ = hf(h, emb, mask)
        actual, _ = hip(h, emb, mask)
    assert torch.equal(actual, expected)


def test_replaced_projection_weight_turns_the_fused_projection_off(device):
    """A q_proj weight replaced after wrapping is the one used: the layer
    falls back to three GEMMs and still matches the HF module."""
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (Qwen3MoeAttention,
                                                                    Qwen3MoeRotaryEmbedding)

    from specfit_amd.runtime import Qwen3AttentionHip

    torch.manual_seed(7)
    cfg = _attention_config(128)
    hf = Qwen3MoeAttention(cfg, layer_idx=0).to(device=device, dtype=torch.bfloat16).eval()
    hf.q_norm = Qwen3RMSNormHip.from_module(hf.q_norm)
    hf.k_norm = Qwen3RMSNormHip.from_module(hf.k_norm)
    hip = Qwen3AttentionHip.from_module(hf)
    assert hip._fused_projection()
    hf.q_proj.weight = torch.nn.Parameter(torch.randn_like(hf.q_proj.weight))
    assert not hip._fused_projection()
    T = 5
    h = torch.randn(1, T, 256, device=device).to(torch.bfloat16)
    emb = Qwen3MoeRotaryEmbedding(cfg).to(device)(h, torch.arange(T, device=device)[None])
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool, device=device)).view(1, 1, T, T)
    with torch.no_grad():
        expected, _ = hf(h, emb, mask)
        actual, _ = hip(h, emb, mask)
    assert torch.equal(actual, expected)


def test_qk_norm_rope_rejects_other_head_dims(device):
    q = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16, device=device)
    w = torch.ones(64, dtype=torch.bfloat16, device=device)
    cs = torch.zeros(1, 2, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError, match="unsupported"):
        ops.qk_norm_rope(q, q, w, w, 1e-6, cs, cs)
