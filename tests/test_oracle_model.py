"""Pin the oracle's config-4 block stack (rms_norm, swiglu, iso/diag layer, GPT) and check the
product modules' structure on the CPU: parameter names and totals against the reference's own
figures, closed-form reductions of the composition, constructor and forward argument checks."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import kdn_oracle as ko


def _tiny(mixer_type, **kw):
    from lit_gpt.config import Config
    base = dict(name="tiny", block_size=256, vocab_size=100, padding_multiple=64, gdn2_per_layer=1,
                mixer_type=mixer_type, n_layer=2, n_head=2, n_embd=128, rotary_percentage=1.0,
                parallel_residual=False, bias=False, _norm_class="FusedRMSNorm", norm_eps=1e-5,
                _mlp_class="LLaMAMLP", intermediate_size=96, mamba_init=True, kdn_info_scale=64.0)
    base.update(kw)
    return Config(**base)


def _params(model):
    return {k: v.detach().double() for k, v in model.state_dict().items()}


def test_rms_norm_matches_torch_rms_norm():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 5, 40, generator=g, dtype=torch.float64)
    w = torch.randn(40, generator=g, dtype=torch.float64)
    assert torch.allclose(ko.rms_norm(x, w, 1e-5), F.rms_norm(x, (40,), w, 1e-5), atol=1e-14, rtol=0)


def test_swiglu_closed_form_and_amp_rounding():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 3, 8, generator=g, dtype=torch.float64)
    eye = torch.eye(8, dtype=torch.float64)
    assert torch.allclose(ko.swiglu(x, eye, eye, eye), F.silu(x) * x, atol=1e-15, rtol=0)
    # under amp every stored value is a bf16 number
    y = ko.swiglu(x, eye, 2 * eye, eye, amp=True)
    assert torch.equal(y, y.to(torch.bfloat16).double())
    assert float((y - 2 * F.silu(x) * x).abs().max()) < 2e-2 * float(y.abs().max())


@pytest.mark.parametrize("name,total,blocks", [("iso_kdn_1.3B", 1_449_848_592, 1_302_390_288),
                                               ("diag_kdn_1.3B", 1_449_806_796, 1_302_348_492)])
def test_config4_parameter_totals_match_reference(name, total, blocks):
    """The reference states both totals beside the configurations (config.py:139,164)."""
    from lit_gpt.model import GPT
    with torch.device("meta"):
        model = GPT.from_name(name)
    assert sum(p.numel() for p in model.parameters()) == total
    assert sum(p.numel() for p in model.transformer.h.parameters()) == blocks
    assert model.config.padded_vocab_size == 32000 and model.config.head_size == 128


def test_layer_state_dict_names_match_reference():
    """Names after the reference's projection packing (iso_kdn_chunk.py:696-729) and the diagonal
    layer's plain modules (diag_kdn.py:183-240)."""
    from lit_gpt.diag_kdn import DiagonalKalmanDeltaNetwork
    from lit_gpt.iso_kdn import IsotropicKalmanDeltaNetwork
    iso = IsotropicKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=2)
    assert {k: tuple(v.shape) for k, v in iso.state_dict().items()} == {
        "qkv_pack.projection_weight": (384, 128), "qkv_pack.convolution_weight": (384, 4),
        "f_omega_r_proj.weight": (68, 128), "f_proj.1.weight": (128, 64), "omega_proj.bias": (2,),
        "r_proj.bias": (2,), "A_log": (2,), "dt_bias": (128,), "g_proj.0.weight": (64, 128),
        "g_proj.1.weight": (128, 64), "g_proj.1.bias": (128,), "o_norm.weight": (64,), "o_proj.weight": (128, 128),
        "initial_precision_param": (2,)}
    diag = DiagonalKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=2)
    assert {k: tuple(v.shape) for k, v in diag.state_dict().items()} == {
        "q_proj.weight": (128, 128), "k_proj.weight": (128, 128), "v_proj.weight": (128, 128),
        "q_conv1d.weight": (128, 1, 4), "k_conv1d.weight": (128, 1, 4), "v_conv1d.weight": (128, 1, 4),
        "f_proj.0.weight": (64, 128), "f_proj.1.weight": (128, 64), "A_log": (2,), "dt_bias": (128,),
        "g_proj.0.weight": (64, 128), "g_proj.1.weight": (128, 64), "g_proj.1.bias": (128,),
        "o_norm.weight": (64,), "o_proj.weight": (128, 128), "omega_proj.0.weight": (64, 128),
        "omega_proj.1.weight": (128, 64), "omega_proj.1.bias": (128,), "r_proj.weight": (2, 128),
        "r_proj.bias": (2,), "initial_precision_param": (2,)}
    # the diagonal layer starts from isotropic process noise; initial precision is 1
    assert not diag.omega_proj[1].weight.any() and not diag.omega_proj[1].bias.any()
    mu = 0.1 + F.softplus(iso.initial_precision_param)
    assert torch.allclose(mu, torch.ones(2))


@pytest.mark.parametrize("mixer_type", ["iso_kdn", "diag_kdn"])
def test_gpt_oracle_closed_form_reductions(mixer_type):
    """Zero o_proj: every block is x + mlp(norm_2(x)); zero o_proj and w3: the logits are
    lm_head(ln_f(wte[idx])).  The oracle composition must reduce exactly."""
    from lit_gpt.model import GPT
    torch.manual_seed(0)
    model = GPT(_tiny(mixer_type))
    model.init_weights()
    p = _params(model)
    idx = torch.randint(0, 100, (1, 9))
    kw = {"info_scale": 64.0} if mixer_type == "iso_kdn" else {}
    for i in range(2):
        p[f"transformer.h.{i}.attn.o_proj.weight"].zero_()
    x = p["transformer.wte.weight"][idx]
    for i in range(2):
        b = f"transformer.h.{i}."
        x = x + ko.swiglu(ko.rms_norm(x, p[b + "norm_2.weight"]), p[b + "mlp.swiglu.w1.weight"],
                          p[b + "mlp.swiglu.w2.weight"], p[b + "mlp.swiglu.w3.weight"])
    ref = ko.rms_norm(x, p["transformer.ln_f.weight"]) @ p["lm_head.weight"].T
    got = ko.gpt_forward(p, idx, n_layer=2, mixer_type=mixer_type, **kw)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)
    for i in range(2):
        p[f"transformer.h.{i}.mlp.swiglu.w3.weight"].zero_()
    ref = ko.rms_norm(p["transformer.wte.weight"][idx], p["transformer.ln_f.weight"]) @ p["lm_head.weight"].T
    got = ko.gpt_forward(p, idx, n_layer=2, mixer_type=mixer_type, **kw)
    assert torch.allclose(got, ref, atol=1e-12, rtol=0)


def test_layer_oracle_is_linear_in_the_output_projection():
    """out = o_proj(y): doubling o_proj doubles the output; y = norm(o) w sigmoid(gate): doubling
    o_norm's weight doubles it too (the gated norm is scale-free in o)."""
    from lit_gpt.iso_kdn import IsotropicKalmanDeltaNetwork
    torch.manual_seed(1)
    p = _params(IsotropicKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=2))
    x = torch.randn(1, 6, 128, dtype=torch.float64)
    y = ko.iso_layer(p, x)
    p2 = dict(p, **{"o_proj.weight": 2 * p["o_proj.weight"]})
    assert torch.allclose(ko.iso_layer(p2, x), 2 * y, atol=1e-12, rtol=0)
    p3 = dict(p, **{"o_norm.weight": 2 * p["o_norm.weight"]})
    assert torch.allclose(ko.iso_layer(p3, x), 2 * y, atol=1e-12, rtol=0)


def test_model_argument_checks():
    from lit_gpt.config import Config
    from lit_gpt.diag_kdn import DiagonalKalmanDeltaNetwork
    from lit_gpt.iso_kdn import IsotropicKalmanDeltaNetwork
    from lit_gpt.model import GPT
    with pytest.raises(ValueError):
        IsotropicKalmanDeltaNetwork(hidden_size=96, head_dim=32, num_heads=3)
    with pytest.raises(ValueError):
        IsotropicKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=3)
    with pytest.raises(ValueError):
        IsotropicKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=2, r_min=0.0)
    with pytest.raises(ValueError):
        DiagonalKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=2, r_min=0.02)
    with pytest.raises(ValueError):
        DiagonalKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=2, info_scale=32.0)
    layer = IsotropicKalmanDeltaNetwork(hidden_size=128, head_dim=64, num_heads=2)
    x = torch.zeros(1, 4, 128)
    with pytest.raises(ValueError, match="CUDA"):
        layer(x)
    with pytest.raises(ValueError, match="fixed-length"):
        layer(x, attention_mask=torch.ones(1, 4))
    with pytest.raises(ValueError, match="sequence length >= 2"):
        layer(torch.zeros(1, 1, 128))
    with pytest.raises(ValueError):
        Config(n_embd=128, n_head=2, _mlp_class="LLaMAMLP")  # needs intermediate_size
    with pytest.raises(ValueError, match="only KDN"):
        GPT(_tiny("gdn2"))
    model = GPT(_tiny("iso_kdn"))
    with pytest.raises(ValueError, match="KV caching"):
        model(torch.zeros(1, 4, dtype=torch.long), input_pos=torch.arange(4))
    assert math.isclose(Config.from_name("iso_kdn_1.3B").kdn_info_scale, 128.0)
