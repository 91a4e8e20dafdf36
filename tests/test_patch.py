"""Host-side behaviour of the patcher and the registration (no GPU needed):
which modules are replaced or routed, that weights keep their storage and
state_dict keys, that the fused ops refuse CPU tensors, and the torch.library
schemas (reference patch.py:92-240, ops/fused_lora.py:323-421,
_torch_library.py:26-86)."""

import pytest
import torch

from tests import qwen_tiny


def test_patch_counts_keys_and_storage():
    from metal_liger_amd import MetalLigerRMSNorm, MetalLigerSwiGLU, apply_metal_liger_to_qwen3vl
    model = qwen_tiny.build()
    keys_before = list(model.state_dict().keys())
    lm = model.base_model.model
    ptr_in = lm.model.layers[0].input_layernorm.weight.data_ptr()
    ptr_final = lm.model.norm.weight.data_ptr()
    out = apply_metal_liger_to_qwen3vl(model)
    assert out is model
    norms = [m for m in model.modules() if isinstance(m, MetalLigerRMSNorm)]
    assert len(norms) == 2 * 2 + 1                     # 2 per layer + the final norm
    assert sum(isinstance(l.mlp, MetalLigerSwiGLU) for l in lm.model.layers) == 2
    assert all(getattr(l.self_attn, "_metal_liger_fused_lora", False) for l in lm.model.layers)
    assert all(getattr(l.mlp, "_metal_liger_fused_lora", False) for l in lm.model.layers)
    assert list(model.state_dict().keys()) == keys_before
    assert lm.model.layers[0].input_layernorm.weight.data_ptr() == ptr_in
    assert lm.model.norm.weight.data_ptr() == ptr_final
    assert "fused=MetalLiger" in repr(lm.model.norm)


def test_patch_bare_model_and_flags():
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    from metal_liger_amd.ops.fused_lora import patch_fused_lora
    lm = qwen_tiny.build(lora=False, peft_wrap=False)
    apply_metal_liger_to_qwen3vl(lm, fuse_swiglu=False, fuse_lora=True, fuse_rope=True,
                                 fuse_cross_entropy=True)
    assert type(lm.model.layers[0].mlp).__name__ == "Qwen3MLP"      # swiglu not fused
    assert patch_fused_lora(lm) == 0                                 # no LoRA adapters
    assert patch_fused_lora(torch.nn.Linear(4, 4)) == 0              # no layers at all


def test_patch_lora_routing_without_replacement():
    from metal_liger_amd.ops.fused_lora import _get_lora_params, patch_fused_lora
    model = qwen_tiny.build()
    lm = model.base_model.model
    q = lm.model.layers[0].self_attn.q_proj
    W, A, B, s = _get_lora_params(q)
    assert W is q.base_layer.weight and A.shape == (16, 128) and B.shape == (128, 16) and s == 2.0
    assert _get_lora_params(torch.nn.Linear(3, 3)) == (None, None, None, None)
    n = patch_fused_lora(model)
    assert n == 4
    assert lm.model.layers[0].self_attn.q_proj is q                  # module not replaced


def test_fused_ops_refuse_cpu_tensors():
    from metal_liger_amd import MetalLigerRMSNorm
    from metal_liger_amd.ops.fused_swiglu import fused_swiglu
    with pytest.raises(ValueError, match="ROCm GPU"):
        MetalLigerRMSNorm(8)(torch.randn(2, 8))
    with pytest.raises(ValueError, match="ROCm GPU"):
        fused_swiglu(torch.randn(4), torch.randn(4))


def test_torch_library_schemas():
    import metal_liger_amd  # noqa: F401  (registers on import)
    ops = torch.ops.metal_liger
    assert "float eps, str kernel_dir" in str(ops.rms_norm_forward.default._schema)
    assert str(ops.swiglu_forward.default._schema).endswith("(Tensor gate, Tensor up, str kernel_dir) -> Tensor")
    from metal_liger_amd._torch_library import register_metal_liger_ops
    register_metal_liger_ops()                                       # idempotent


def test_reference_import_paths():
    import metal_liger
    from metal_liger.ops.fused_rope import _rotate_half, apply_fused_rotary  # noqa: F401
    from metal_liger.ops.fused_linear_cross_entropy import MetalLigerFusedLinearCrossEntropy  # noqa: F401
    import metal_liger_ext
    assert set(metal_liger.__all__) >= {
        "MetalLigerRMSNorm", "MetalLigerSwiGLU", "MetalLigerRoPE", "MetalLigerFusedLinearCrossEntropy",
        "apply_metal_liger_to_qwen3vl", "apply_fused_lora_qkv", "apply_fused_lora_mlp",
        "patch_fused_lora", "apply_compile", "register_metal_liger_ops"}
    assert metal_liger.__version__ == "0.3.0"
    for f in ("rms_norm_forward", "rms_norm_backward", "swiglu_forward", "swiglu_backward"):
        assert callable(getattr(metal_liger_ext, f))
    m = torch.nn.Linear(2, 2)
    assert metal_liger.apply_compile(m) is m
