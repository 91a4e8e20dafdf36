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
    keys = list(lm.state_dict())
    apply_metal_liger_to_qwen3vl(lm, fuse_swiglu=False, fuse_lora=True, fuse_rope=True,
                                 fuse_cross_entropy=True)
    assert type(lm.model.layers[0].mlp).__name__ == "Qwen3MLP"      # swiglu not fused
    # fuse_rope / fuse_cross_entropy only log, as in the reference (patch.py:226-232)
    attn = lm.model.layers[0].self_attn
    assert not getattr(attn, "_metal_liger_qk_norm_rope", False)
    assert not getattr(lm, "_metal_liger_flce_loss", False)
    assert "forward" not in lm.__dict__ and "forward" not in attn.__dict__
    assert list(lm.state_dict()) == keys
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
    keys = list(model.state_dict())
    n = patch_fused_lora(model)
    assert n == 4
    assert patch_fused_lora(model) == 0                              # already routed
    assert lm.model.layers[0].self_attn.q_proj is q                  # module not replaced
    assert list(model.state_dict()) == keys


class _Block(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = torch.nn.Module()
        self.mlp = torch.nn.Module()


def test_layer_search_paths_and_fallback():
    """The decoder layers are found along the wrapping layouts (bare decoder,
    causal LM, PEFT, Qwen3-VL) and, for any other wrapper, as the first
    non-empty ModuleList named ``layers``."""
    from metal_liger_amd._model_walk import find_layers
    model = qwen_tiny.build()
    assert find_layers(model) is model.base_model.model.model.layers
    assert find_layers(model.base_model.model) is model.base_model.model.model.layers
    assert find_layers(model.base_model.model.model) is model.base_model.model.model.layers
    outer = torch.nn.Module()
    outer.wrapped = torch.nn.Module()
    outer.wrapped.inner = torch.nn.Module()
    outer.wrapped.inner.layers = torch.nn.ModuleList([_Block(), _Block()])
    assert find_layers(outer) is outer.wrapped.inner.layers
    outer.wrapped.inner.layers = torch.nn.ModuleList()
    assert find_layers(outer) is None


def test_shadowed_restores_instance_dict():
    """shadowed() hides submodules for the duration of a block only, and puts
    back an instance attribute that was there before, also on an error."""
    from metal_liger_amd._model_walk import shadowed
    m = torch.nn.Module()
    m.proj = torch.nn.Linear(2, 2)
    m.__dict__["tag"] = "old"
    with shadowed(m, proj="p", tag="new"):
        assert m.proj == "p" and m.tag == "new"
    assert isinstance(m.proj, torch.nn.Linear) and m.tag == "old"
    with pytest.raises(KeyError):
        with shadowed(m, proj="p"):
            raise KeyError("x")
    assert isinstance(m.proj, torch.nn.Linear) and "proj" not in m.__dict__


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


def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1):
    """Module-level rotary of this test file, for _NoRotaryAttention below."""
    return q, k


class _NoRotaryAttention(torch.nn.Module):
    """An attention-like module with q_norm / k_norm whose forward never
    reaches apply_rotary_pos_emb."""

    def __init__(self, d=32):
        super().__init__()
        from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
        self.q_proj = torch.nn.Linear(d, d)
        self.q_norm = Qwen3RMSNorm(d)
        self.k_norm = Qwen3RMSNorm(d)
        self.head_dim = d

    def forward(self, x):
        return self.q_norm(self.q_proj(x))


def test_qk_norm_rope_patch_defers_norms_to_the_rotary_step(monkeypatch):
    """fuse_qk_norm_rope routes Qwen3 attention's q_norm / k_norm into the rotary step
    of the same forward. With the fused op swapped for the oracle on the CPU,
    the patched model's logits equal the unpatched model's bit for bit, an
    unpatched instance in the same process keeps transformers' own rotary,
    and a forward that never reaches the rotary raises."""
    import copy

    import metal_liger_amd.ops.fused_qk_norm_rope as fq
    from oracle import reference_ops as ref
    calls = []

    def oracle_fused(q, k, q_norm, k_norm, cos, sin, unsqueeze_dim=1):
        calls.append(q.shape)
        c, s = cos.unsqueeze(unsqueeze_dim), sin.unsqueeze(unsqueeze_dim)
        return (ref.qk_norm_rope_forward(q, q_norm.weight, q_norm.variance_epsilon, c, s),
                ref.qk_norm_rope_forward(k, k_norm.weight, k_norm.variance_epsilon, c, s))

    monkeypatch.setattr(fq, "apply_fused_qk_norm_rope", oracle_fused)
    lm = qwen_tiny.build(seed=5, lora=False, peft_wrap=False)
    with torch.no_grad():
        for layer in lm.model.layers:           # non-trivial norm weights
            layer.self_attn.q_norm.weight.normal_(1.0, 0.1)
            layer.self_attn.k_norm.weight.normal_(1.0, 0.1)
    other = copy.deepcopy(lm)
    ids = torch.randint(0, 512, (2, 24), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        want = lm(input_ids=ids).logits
    keys = list(lm.state_dict())
    assert fq.patch_qk_norm_rope(lm) == 2
    assert fq.patch_qk_norm_rope(lm) == 0                            # idempotent
    assert list(lm.state_dict()) == keys
    with torch.no_grad():
        got = lm(input_ids=ids).logits
        got_other = other(input_ids=ids).logits
    assert calls == [(2, 4, 24, 32)] * 2                             # one call per layer
    assert torch.equal(got, want)
    assert torch.equal(got_other, want)
    assert "q_norm" not in lm.model.layers[0].self_attn.__dict__     # shadow removed

    bad = _NoRotaryAttention()
    assert fq.patch_qk_norm_rope(bad) == 1
    with pytest.raises(RuntimeError, match="did not call apply_rotary_pos_emb"):
        bad(torch.randn(2, 32))


class _OracleAddNorm:
    """Stand-in for the fused residual add + norm Function on the CPU."""

    calls = 0

    @staticmethod
    def apply(x, residual, weight, eps):
        from oracle import reference_ops as ref
        _OracleAddNorm.calls += 1
        y, total, _ = ref.add_rms_norm_forward(x, residual, weight, eps)
        return y, total


class _ExtraAddLayer(torch.nn.Module):
    """Has the four parts of a decoder layer but a third addition: not the
    structure the fused forward reproduces, so it must stay unpatched."""

    def __init__(self):
        super().__init__()
        from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm
        self.input_layernorm = MetalLigerRMSNorm(8)
        self.self_attn = torch.nn.Identity()
        self.post_attention_layernorm = MetalLigerRMSNorm(8)
        self.mlp = torch.nn.Identity()

    def forward(self, hidden_states):
        residual = hidden_states
        h = self.self_attn(self.input_layernorm(hidden_states))
        h = residual + h + 1.0
        residual = h
        h = self.mlp(self.post_attention_layernorm(h))
        return residual + h


class _TupleReturnLayer(_ExtraAddLayer):
    """transformers' older decoder-layer form: returns an outputs tuple and
    appends to it with +=."""

    def forward(self, hidden_states, output_attentions=False):
        residual = hidden_states
        h = self.self_attn(self.input_layernorm(hidden_states))
        h = residual + h
        residual = h
        h = self.mlp(self.post_attention_layernorm(h))
        h = residual + h
        outputs = (h,)
        if output_attentions:
            outputs += (None,)
        return outputs


class _BareTupleLayer(_ExtraAddLayer):
    def forward(self, hidden_states):
        residual = hidden_states
        h = self.self_attn(self.input_layernorm(hidden_states))
        h = residual + h
        residual = h
        h = self.mlp(self.post_attention_layernorm(h))
        return (residual + h,)


def test_residual_add_norm_patch_matches_unfused(monkeypatch):
    """fuse_residual_norm swaps each Qwen3 decoder layer's forward for one
    that fuses the post-attention add into post_attention_layernorm. With the
    fused norms swapped for the oracle on the CPU, logits and gradients equal
    the unfused model's bit for bit (every argument reaches the attention as
    before); layers of another structure, or whose norm is not the fused
    norm, are left alone."""
    import copy

    import metal_liger_amd.ops.fused_add_rms_norm as fa
    from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm
    from metal_liger_amd.patch import apply_metal_liger_to_qwen3vl
    from oracle import reference_ops as ref

    monkeypatch.setattr(MetalLigerRMSNorm, "forward",
                        lambda self, x: ref.rms_norm_forward(x, self.weight, self.eps)[0])
    monkeypatch.setattr(fa, "_FusedAddRMSNormFunction", _OracleAddNorm)
    base = qwen_tiny.build(seed=6, lora=False, peft_wrap=False)
    assert fa.patch_residual_add_norm(base) == 0                    # HF norms: not eligible
    kw = dict(fuse_swiglu=False, fuse_lora=False)
    unfused = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), **kw)
    fused = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), fuse_residual_norm=True, **kw)
    assert all(getattr(layer, "_metal_liger_add_norm", False) for layer in fused.model.layers)
    assert list(fused.state_dict()) == list(unfused.state_dict())
    assert fa.patch_residual_add_norm(fused) == 0                   # idempotent

    ids = torch.randint(0, 512, (2, 20), generator=torch.Generator().manual_seed(3))
    outs = []
    for m in (unfused, fused):
        m.zero_grad()
        logits = m(input_ids=ids).logits
        logits.float().square().mean().backward()
        outs.append((logits.detach(), {n: p.grad.clone() for n, p in m.named_parameters()}))
    assert _OracleAddNorm.calls == 2                                # one per layer
    assert torch.equal(outs[0][0], outs[1][0])
    for n, g in outs[0][1].items():
        assert torch.equal(outs[1][1][n], g), n

    assert fa.patch_residual_add_norm(_ExtraAddLayer()) == 0
    assert fa.patch_residual_add_norm(_TupleReturnLayer()) == 0      # returns a tuple
    assert fa.patch_residual_add_norm(_BareTupleLayer()) == 0
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextDecoderLayer
    for cls in (Qwen3DecoderLayer, Qwen3VLTextDecoderLayer):
        assert fa._structure(cls.forward) == (fa._LAYER_PARTS, 2, True)


class _OracleFLCE:
    """Stand-in for the fused loss's autograd Function on the CPU: the
    oracle's chunked CE (mean over valid tokens, 0 when none is valid)."""

    calls = 0

    @staticmethod
    def apply(h, w, y, b, ignore_index, chunk_size):
        from oracle import reference_ops as ref
        _OracleFLCE.calls += 1
        loss, _, _ = ref.flce_forward(h, w, y, b, ignore_index, chunk_size)
        return loss


class _OracleCops:
    """Stand-in for the custom-op module as the fused loss calls it with
    grad mode off: the loss-only op, answered by the oracle."""

    @staticmethod
    def flce_fwd(h, w, y, b, ignore_index, chunk_size):
        from oracle import reference_ops as ref
        _OracleFLCE.calls += 1
        loss, lse, mask = ref.flce_forward(h, w, y, b, ignore_index, chunk_size)
        return loss, lse, mask.sum().float().reshape(1)


class _RecordingCops:
    """Records which FLCE entry point the fused loss called (no compute)."""

    def __init__(self):
        self.calls = []

    def flce_fwd(self, h, w, y, b, ignore_index, chunk_size):
        self.calls.append(("flce_fwd", h.dtype))
        return torch.zeros(()), torch.zeros(h.shape[0]), torch.ones(1)

    def flce_fwd_grad(self, h, w, y, b, ignore_index, need_h, need_w, chunk_size):
        self.calls.append(("flce_fwd_grad", need_h, need_w))
        e = torch.empty(0)
        return (torch.zeros(()), torch.zeros(h.shape[0]), torch.ones(1),
                torch.zeros_like(h) if need_h else e, torch.zeros_like(w) if need_w else e)

    @staticmethod
    def maybe(t):
        return None if t.dim() == 1 and t.shape[0] == 0 else t

    def flce_scale_grads(self, g, dh, dw):
        self.calls.append(("flce_scale_grads",))


class _RecordingLoraCops:
    """Stand-in for the custom-op module in the bf16 LoRA MLP Function:
    outputs of the right shapes, and the h its backward is called with."""

    def __init__(self):
        self.h = "not called"

    def lora_xa(self, x, a):
        return torch.zeros(x.shape[0], a.shape[0], dtype=torch.bfloat16)

    def lora_linear_out(self, x, w, xa, sb):
        return torch.zeros(x.shape[0], w.shape[0], dtype=torch.bfloat16)

    def swiglu_fwd(self, g, u):
        return torch.zeros_like(g)

    def lora_mlp_bwd(self, x2, gate, up, h, dy, *rest):
        from metal_liger_amd import hip_ops
        self.h = h
        shapes = hip_ops.lora_mlp_grad_shapes(x2.shape[1], gate.shape[1], rest[-1])
        return torch.zeros_like(x2), torch.zeros(hip_ops.grad_layout(shapes)[1])


def test_lora_mlp_saves_no_h_and_recomputes_it(monkeypatch):
    """The bf16 MLP Function keeps gate and up for its backward but not
    h = silu(gate) up (the reference saves all three,
    ops/fused_lora.py:197-204), and calls the fused backward with h = None:
    the kernels recompute h with the SwiGLU forward's math."""
    import metal_liger_amd.ops.fused_lora as fl
    rec = _RecordingLoraCops()
    monkeypatch.setattr(fl, "cops", rec)
    N, H, I, r = 24, 32, 48, 8
    bf = torch.bfloat16

    def adapter(o, i):
        return (torch.randn(o, i, dtype=bf), torch.randn(r, i, dtype=bf, requires_grad=True),
                torch.randn(o, r, dtype=bf, requires_grad=True), 2.0)

    X = torch.randn(N, H, dtype=bf, requires_grad=True)
    out = fl._LoRA_MLP.apply(X, *adapter(I, H), *adapter(I, H), *adapter(H, I))
    saved = out.grad_fn.saved_tensors
    assert sum(1 for t in saved if tuple(t.shape) == (N, I)) == 2  # gate and up only
    out.backward(torch.ones_like(out))
    assert rec.h is None and X.grad is not None


def test_fused_loss_routes_no_grad_to_loss_only(monkeypatch):
    """With grad mode off the module (and the causal-LM loss) call the
    loss-only entry point even when the lm_head weight requires grad; with
    grad mode on, the autograd Function's one-pass forward + gradients."""
    import metal_liger_amd.ops.fused_linear_cross_entropy as fl
    rec = _RecordingCops()
    monkeypatch.setattr(fl, "cops", rec)
    head = torch.nn.Linear(16, 40, bias=False)
    assert head.weight.requires_grad
    mod = fl.MetalLigerFusedLinearCrossEntropy(head)
    h = torch.randn(2, 5, 16, requires_grad=True)
    y = torch.randint(0, 40, (2, 5))
    with torch.no_grad():
        mod(h, y)
    assert rec.calls == [("flce_fwd", torch.float32)]
    with torch.inference_mode():
        fl.causal_lm_loss(h.detach(), head, y)
    assert rec.calls[-1] == ("flce_fwd", torch.float32) and len(rec.calls) == 2
    # fp16 operands are upcast to fp32 before the loss-only op, as for the Function
    with torch.no_grad():
        fl.MetalLigerFusedLinearCrossEntropy(head.half())(h.half(), y)
    assert rec.calls[-1] == ("flce_fwd", torch.float32)
    head.float()
    rec.calls.clear()
    loss = mod(h, y)
    assert rec.calls == [("flce_fwd_grad", True, True)]
    loss.backward()
    assert rec.calls[-1] == ("flce_scale_grads",)
    rec.calls.clear()
    head.weight.requires_grad_(False)
    mod(h, y)
    assert rec.calls == [("flce_fwd_grad", True, False)]


def test_causal_lm_loss_hook_matches_transformers(monkeypatch):
    """fuse_lm_loss routes a causal LM's training loss through the fused
    op with transformers' label shift; the logits are not returned; with
    num_items_in_batch the sum is divided by it; eval mode is unchanged."""
    import copy

    import metal_liger_amd.ops.fused_linear_cross_entropy as fl
    monkeypatch.setattr(fl, "_FusedLinearCrossEntropyFunction", _OracleFLCE)
    monkeypatch.setattr(fl, "cops", _OracleCops)  # grad mode is off below: the loss-only op
    lm = qwen_tiny.build(seed=6, lora=False, peft_wrap=False)
    ref_lm = copy.deepcopy(lm)
    ids = torch.randint(0, 512, (2, 20), generator=torch.Generator().manual_seed(3))
    labels = ids.clone()
    labels[0, :5] = -100
    lm.train()
    ref_lm.train()
    assert fl.patch_causal_lm_loss(lm) == 1
    assert fl.patch_causal_lm_loss(lm) == 0                          # idempotent
    with torch.no_grad():
        want = ref_lm(input_ids=ids, labels=labels)
        got = lm(input_ids=ids, labels=labels)
        n_items = torch.tensor(50.0)
        want_n = ref_lm(input_ids=ids, labels=labels, num_items_in_batch=n_items).loss
        got_n = lm(input_ids=ids, labels=labels, num_items_in_batch=n_items).loss
    assert _OracleFLCE.calls == 2 and got.logits is None
    assert torch.allclose(got.loss, want.loss, rtol=1e-5, atol=1e-6)
    assert torch.allclose(got_n, want_n, rtol=1e-5, atol=1e-6)
    assert "lm_head" not in lm.__dict__ and "_loss_function" not in lm.__dict__
    lm.eval()                                                        # eval: transformers' path
    with torch.no_grad():
        ev = lm(input_ids=ids, labels=labels)
    assert ev.logits is not None and _OracleFLCE.calls == 2
    assert torch.allclose(ev.loss, want.loss, rtol=1e-5, atol=1e-6)


class _OracleSwiGLU:
    """Stand-in for the fused SwiGLU Function on the CPU."""

    @staticmethod
    def apply(gate, up):
        from oracle import reference_ops as ref
        return ref.swiglu_forward(gate, up)[0]


def test_qwen3_vl_text_stack_patched(monkeypatch):
    """apply_metal_liger_to_qwen3vl on a Qwen3-VL model (the reference's
    target, patch.py:181-240): the language model's layer and final norms,
    MLPs, q/k norms + RoPE, post-attention add + norm and the training loss
    are routed, the vision tower is left alone, state_dict keys are
    unchanged; with every fused op swapped for the oracle on the CPU, the
    loss and all gradients match the unpatched model (fp32 bar: the fused
    loss is the chunked CE, SwiGLU the reference's sigmoid form)."""
    import copy

    import metal_liger_amd.ops.fused_add_rms_norm as fa
    import metal_liger_amd.ops.fused_linear_cross_entropy as fl
    import metal_liger_amd.ops.fused_qk_norm_rope as fq
    import metal_liger_amd.ops.fused_swiglu as fs
    from metal_liger_amd import MetalLigerRMSNorm, MetalLigerSwiGLU, apply_metal_liger_to_qwen3vl
    from oracle import reference_ops as ref

    def oracle_qkn(q, k, q_norm, k_norm, cos, sin, unsqueeze_dim=1):
        c, s = cos.unsqueeze(unsqueeze_dim), sin.unsqueeze(unsqueeze_dim)
        return (ref.qk_norm_rope_forward(q, q_norm.weight, q_norm.variance_epsilon, c, s),
                ref.qk_norm_rope_forward(k, k_norm.weight, k_norm.variance_epsilon, c, s))

    monkeypatch.setattr(MetalLigerRMSNorm, "forward",
                        lambda self, x: ref.rms_norm_forward(x, self.weight, self.eps)[0])
    monkeypatch.setattr(fs, "_FusedSwiGLUFunction", _OracleSwiGLU)
    monkeypatch.setattr(fq, "apply_fused_qk_norm_rope", oracle_qkn)
    monkeypatch.setattr(fa, "_FusedAddRMSNormFunction", _OracleAddNorm)
    monkeypatch.setattr(fl, "_FusedLinearCrossEntropyFunction", _OracleFLCE)

    base = qwen_tiny.build_vl(seed=8)
    keys = list(base.state_dict())
    patched = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), fuse_qk_norm_rope=True,
                                           fuse_lm_loss=True, fuse_residual_norm=True)
    lm = patched.model.language_model
    assert sum(isinstance(m, MetalLigerRMSNorm) for m in patched.modules()) == 2 * 2 + 1
    assert all(isinstance(layer.mlp, MetalLigerSwiGLU) for layer in lm.layers)
    assert all(getattr(layer.self_attn, "_metal_liger_qk_norm_rope", False) for layer in lm.layers)
    assert all(getattr(layer, "_metal_liger_add_norm", False) for layer in lm.layers)
    assert getattr(patched, "_metal_liger_flce_loss", False)
    assert not any(isinstance(m, (MetalLigerRMSNorm, MetalLigerSwiGLU))
                   for m in patched.model.visual.modules())
    assert list(patched.state_dict()) == keys

    ids = torch.randint(0, 512, (2, 24), generator=torch.Generator().manual_seed(4))
    results = []
    for m in (base, patched):
        m.train()
        m.zero_grad()
        out = m(input_ids=ids, labels=ids)
        out.loss.backward()
        results.append((out.loss.detach(), {n: p.grad for n, p in m.named_parameters()
                                            if p.grad is not None}))
    (l0, g0), (l1, g1) = results
    assert torch.allclose(l1, l0, rtol=1e-5, atol=1e-6), (l1, l0)
    assert set(g1) == set(g0) and len(g0) > 0
    for n, g in g0.items():
        err = (g1[n].double() - g.double()).abs().max()
        assert err <= 1e-4 * g.double().abs().max() + 1e-7, n


def test_efficient_attention_matches_sdpa():
    """efficient_attention=True (key / value heads repeated, SDPA with the
    memory-efficient kernel first) against transformers' own "sdpa" path on
    the tiny GQA model (4 query / 2 key-value heads), fp32 on the CPU: the
    causal case (no mask tensor) and a left-padded batch (a mask tensor);
    a model on "eager" keeps it."""
    import copy

    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    from metal_liger_amd.ops.gqa_attention import ATTN_KEY, _repeat_heads
    base = qwen_tiny.build(lora=False, peft_wrap=False, attn="sdpa")
    base.eval()
    patched = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), fuse_rms_norm=False,
                                           fuse_swiglu=False, fuse_lora=False,
                                           efficient_attention=True)
    assert patched.config._attn_implementation == ATTN_KEY
    assert base.config._attn_implementation == "sdpa"
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 512, (2, 24), generator=g)
    mask = torch.ones(2, 24, dtype=torch.long)
    mask[1, :7] = 0
    with torch.no_grad():
        for kw in ({}, {"attention_mask": mask}):
            ref = base(input_ids=ids, use_cache=False, **kw).logits
            out = patched(input_ids=ids, use_cache=False, **kw).logits
            keep = slice(None) if not kw else (mask[:, :, None] > 0).expand_as(ref)
            assert torch.allclose(out[keep], ref[keep], rtol=1e-4, atol=1e-4), kw
        # decoding with a key / value cache: a prompt, then one token per call
        logits = []
        for m in (base, patched):
            o = m(input_ids=ids[:, :20], attention_mask=mask[:, :20], use_cache=True)
            past, step = o.past_key_values, []
            for t in range(20, 24):
                o = m(input_ids=ids[:, t:t + 1], attention_mask=mask[:, :t + 1],
                      past_key_values=past, use_cache=True)
                past = o.past_key_values
                step.append(o.logits[:, -1])
            logits.append(torch.stack(step))
        assert torch.allclose(logits[1], logits[0], rtol=1e-4, atol=1e-4)
    # query head h reads key / value head h // groups
    kv = torch.arange(2 * 3, dtype=torch.float32).reshape(1, 3, 2, 1)
    rep = _repeat_heads(kv, 2)
    assert rep.shape == (1, 6, 2, 1)
    assert torch.equal(rep[0, :, 0, 0], torch.tensor([0.0, 0.0, 2.0, 2.0, 4.0, 4.0]))
    eager = qwen_tiny.build(lora=False, peft_wrap=False, attn="eager")
    from metal_liger_amd.ops.gqa_attention import patch_efficient_attention
    assert patch_efficient_attention(eager) == 0
    assert eager.config._attn_implementation == "eager"
    assert patch_efficient_attention(patched) == 2                   # both layers
