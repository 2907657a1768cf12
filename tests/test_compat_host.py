"""Host tests of the drop-in module mirror (rldx_amd.compat): after install(),
the module names the reference's chains import resolve to the rldx_amd
launchers, with the reference's function names, parameter names and defaults
(each expected signature below is copied from the reference file cited), the
op-registration modules bind the rldx_amd operators, and the set-up helpers
follow their closed forms.  No compute calls: those are in
tests/test_gpu_compat.py."""

import inspect
import sys

import pytest
import torch

from rldx_amd import compat


@pytest.fixture
def installed():
    yield compat.install()
    compat.uninstall()


# (module name as the reference imports it, function, reference parameters as (name, default), citation)
_EMPTY = inspect.Parameter.empty
SIGNATURES = [
    ("double_stream.engine.kernels.vl_epilogue_ln", "fused_vl_epilogue_ln",
     [("vl_residual", _EMPTY), ("proj_bias", _EMPTY), ("w3_bias", _EMPTY), ("w3_out", _EMPTY), ("M", None),
      ("DIM", None), ("new_vl_out", None), ("ln_vl_out", None)], "vl_epilogue_ln.py:134-136"),
    ("double_stream.engine.kernels.grouped_res_ln", "fused_grouped_res_ln",
     [("sa_residual", _EMPTY), ("sa_proj_bias", _EMPTY), ("sa_proj_out", _EMPTY), ("vl_residual", _EMPTY),
      ("vl_proj_bias", _EMPTY), ("vl_proj_out", _EMPTY), ("M_sa", None), ("M_vl", None), ("SA_DIM", None),
      ("VL_DIM", None)], "grouped_res_ln.py:150-161"),
    ("double_stream.engine.kernels.grouped_swiglu", "fused_grouped_swiglu",
     [("sa_w12_out", _EMPTY), ("sa_bias", _EMPTY), ("vl_w12_out", _EMPTY), ("vl_bias", _EMPTY), ("M_sa", None),
      ("M_vl", None), ("N_half_sa", None), ("N_half_vl", None)], "grouped_swiglu.py:213-215"),
    ("single_stream.engine.kernels.ss_epilogue_ln", "fused_ss_epilogue_ln",
     [("hidden", _EMPTY), ("M", None), ("DIM", None), ("residual", None), ("new_hidden_out", None),
      ("ln_out_out", None)], "ss_epilogue_ln.py:146-148"),
    ("single_stream.engine.kernels.fused_mlp_swiglu", "fused_mlp_swiglu",
     [("x", _EMPTY), ("weight", _EMPTY), ("bias", _EMPTY), ("split_k", 1)], "fused_mlp_swiglu.py:199"),
    ("llm.engine.kernels.fused_llm_attention", "forward",
     [("qkv", _EMPTY), ("q_norm_w", _EMPTY), ("q_norm_w_rot", _EMPTY), ("k_norm_w", _EMPTY),
      ("k_norm_w_rot", _EMPTY), ("cos", _EMPTY), ("signed_sin", _EMPTY), ("num_heads", 32), ("num_kv_heads", 8),
      ("head_dim", 128), ("out", None)], "fused_llm_attention.py:1005-1017"),
    ("llm.engine.kernels.fused_llm_attention", "prepare_signed_sin", [("sin", _EMPTY), ("head_dim", _EMPTY)],
     "fused_llm_attention.py:787"),
    ("llm.engine.kernels.fused_llm_attention", "prepare_norm_weight_rot",
     [("norm_weight", _EMPTY), ("head_dim", _EMPTY)], "fused_llm_attention.py:798"),
    ("llm.engine.kernels.fused_llm_attention", "prepare_fused_qkv_weight", [("layer", _EMPTY)],
     "fused_llm_attention.py:778"),
    ("llm.engine.kernels.fused_llm_attention", "autotune_split_m_threshold",
     [("workloads", _EMPTY), ("candidates", (64, 128, 256, 512)), ("warmup", 3), ("iters", 10)],
     "fused_llm_attention.py:928"),
    ("backbone.llm.engine.kernels.fused_add2_rmsnorm", "forward",
     [("hidden", _EMPTY), ("residual", _EMPTY), ("weight", _EMPTY)], "fused_add2_rmsnorm.py:85"),
    ("llm.engine.kernels.fused_add3_rmsnorm", "forward",
     [("hidden", _EMPTY), ("residual", _EMPTY), ("deepstack", _EMPTY), ("weight", _EMPTY)],
     "fused_add3_rmsnorm.py:86"),
    ("vision_encoder.engine.kernels.fused_vision_attention", "forward",
     [("qkv", _EMPTY), ("rope_cos", _EMPTY), ("rope_sin", _EMPTY), ("cu_seqlens", _EMPTY), ("scaling", _EMPTY),
      ("num_heads", _EMPTY), ("head_dim", _EMPTY)], "fused_vision_attention.py:622"),
    ("vision_encoder.engine.kernels.fused_vision_attention", "autotune_split_m_threshold",
     [("workloads", _EMPTY), ("candidates", (64, 128, 256, 512)), ("warmup", 3), ("iters", 10)],
     "fused_vision_attention.py:576"),
    ("memory.engine.kernels.fused_memory_attention", "forward",
     [("qkv", _EMPTY), ("cos", _EMPTY), ("signed_sin", _EMPTY), ("num_heads", _EMPTY), ("head_dim", _EMPTY),
      ("block_attn_size", _EMPTY)], "fused_memory_attention.py:228"),
    ("memory.engine.kernels.fused_memory_attention", "prepare_rope_buffers",
     [("rotary_emb", _EMPTY), ("position_ids", _EMPTY), ("device", _EMPTY), ("dtype", torch.bfloat16)],
     "fused_memory_attention.py:206"),
    ("memory.engine.kernels.fused_memory_attention", "prepare_signed_sin", [("sin", _EMPTY), ("head_dim", _EMPTY)],
     "fused_memory_attention.py:194"),
    ("memory.engine.kernels.fused_add2_rmsnorm", "forward",
     [("hidden", _EMPTY), ("residual", _EMPTY), ("weight", _EMPTY)], "memory/.../fused_add2_rmsnorm.py:15"),
    ("action_model.engine.custom_action_model_chain", "build_custom_action_model_chain",
     [("action_head_model", _EMPTY), ("device", _EMPTY), ("dtype", torch.bfloat16)],
     "custom_action_model_chain.py:174"),
    ("engine.custom_action_model_chain", "compile_custom_action_model_chain",
     [("chain", _EMPTY), ("sample_inputs", _EMPTY), ("compile_mode", "max-autotune"), ("fullgraph", True)],
     "custom_action_model_chain.py:179-181"),
    ("action_model.engine.custom_expanded_action_model_chain", "build_custom_expanded_action_model_chain",
     [("action_head_model", _EMPTY), ("device", _EMPTY), ("dtype", torch.bfloat16)],
     "custom_expanded_action_model_chain.py:216"),
    ("engine.custom_expanded_action_model_chain", "compile_custom_expanded_action_model_chain",
     [("chain", _EMPTY), ("sample_inputs", _EMPTY), ("compile_mode", "max-autotune"), ("fullgraph", True)],
     "custom_expanded_action_model_chain.py:221-223"),
]


CHAIN_FORWARDS = [
    ("engine.custom_action_model_chain", "CustomActionHeadChain",
     ["vl_embs", "state", "embodiment_id", "init_noise", "prefix_actions"], "custom_action_model_chain.py:81-83"),
    ("engine.custom_expanded_action_model_chain", "CustomExpandedActionHeadChain",
     ["vl_embs", "state", "embodiment_id", "init_noise", "physics_hist", "physics_init_noise", "prefix_actions"],
     "custom_expanded_action_model_chain.py:82-91"),
]


@pytest.mark.parametrize("module,cls,params,cite", CHAIN_FORWARDS, ids=[c for _, c, _, _ in CHAIN_FORWARDS])
def test_action_head_chain_signatures(installed, module, cls, params, cite):
    """The mirrored chains take the reference's constructor and forward arguments."""
    c = getattr(sys.modules[module], cls)
    assert list(inspect.signature(c.__init__).parameters)[1:] == ["gs_action_model", "device", "dtype"], cite
    got = [p for p in inspect.signature(c.forward).parameters.values() if p.kind != p.VAR_KEYWORD]
    assert [p.name for p in got[1:]] == params, cite


@pytest.mark.parametrize("module,fn,params,cite", SIGNATURES, ids=[f"{m}.{f}" for m, f, _, _ in SIGNATURES])
def test_launcher_signature_matches_reference(installed, module, fn, params, cite):
    """The reference's parameters, in order and with its defaults, lead the
    mirrored signature; anything after them is an optional keyword."""
    f = getattr(sys.modules[module], fn)
    got = list(inspect.signature(f).parameters.values())
    assert [(p.name, p.default) for p in got[: len(params)]] == params, cite
    assert all(p.default is not _EMPTY for p in got[len(params):]), cite


def test_chain_import_forms_resolve_to_the_mirror(installed):
    """The import statements of the reference's chains, verbatim in form."""
    from backbone.llm.engine.kernels.fused_add2_rmsnorm import forward  # memory/engine/kernels/fused_add2_rmsnorm.py:15
    from double_stream.engine.kernels.vl_epilogue_ln import fused_vl_epilogue_ln  # custom_double_stream_chain.py:12
    from llm.engine.kernels.fused_llm_attention import (  # custom_backbone_chain.py:21-25
        autotune_split_m_threshold, prepare_norm_weight_rot, prepare_signed_sin)
    from single_stream.engine.kernels.ss_epilogue_ln import fused_ss_epilogue_ln  # custom_single_stream_chain.py:11
    from vision_encoder.engine.kernels.fused_vision_attention import autotune_split_m_threshold as v_tune  # :29-31

    import double_stream.engine.ops  # noqa: F401  custom_double_stream_chain.py (ops registration)
    import memory.engine.ops  # noqa: F401  custom_memory_chain.py:18
    import single_stream.engine.ops  # noqa: F401
    for f in (forward, fused_vl_epilogue_ln, autotune_split_m_threshold, prepare_norm_weight_rot, prepare_signed_sin,
              fused_ss_epilogue_ln, v_tune):
        assert f.__module__.startswith("rldx_amd."), f
    assert sys.modules["rldx.inference.action_model.double_stream.engine.kernels.vl_epilogue_ln"] is \
        sys.modules["double_stream.engine.kernels.vl_epilogue_ln"]
    assert autotune_split_m_threshold([]) == 128 and v_tune([]) == 128
    from action_model.engine.custom_action_model_chain import build_custom_action_model_chain  # custom_vla_chain.py:15
    from action_model.engine.custom_expanded_action_model_chain import (  # custom_vla_chain.py:16-18
        build_custom_expanded_action_model_chain)
    from engine.custom_action_model_chain import CustomActionHeadChain  # benchmark_action_model.py:426
    from engine.custom_expanded_action_model_chain import CustomExpandedActionHeadChain  # :419
    for f in (build_custom_action_model_chain, build_custom_expanded_action_model_chain, CustomActionHeadChain,
              CustomExpandedActionHeadChain):
        assert f.__module__.startswith("rldx_amd."), f


OP_MODULES = [
    ("double_stream.engine.ops.op_fused_attention", "fused_attention", "ds::fused_attention_2way"),
    ("double_stream.engine.ops.op_fused_attention_3way", "fused_attention_3way", "ds::fused_attention_3way"),
    ("double_stream.engine.ops.op_vl_epilogue_ln", "vl_epilogue_ln", "ds::vl_epilogue_ln"),
    ("double_stream.engine.ops.op_grouped_swiglu", "grouped_swiglu", "ds::grouped_swiglu"),
    ("double_stream.engine.ops.op_grouped_res_ln", "grouped_res_ln", "ds::grouped_res_ln"),
    ("single_stream.engine.ops.op_fused_attention", "fused_attention", "ss::fused_attention_2way"),
    ("single_stream.engine.ops.op_fused_attention_3way", "fused_attention_3way", "ss::fused_attention_3way"),
    ("single_stream.engine.ops.op_fused_epilogue_ln", "fused_epilogue_ln", "ss::fused_epilogue_ln"),
    ("single_stream.engine.ops.op_fused_mlp_swiglu", "fused_mlp_swiglu", "ss::fused_mlp_swiglu"),
    ("llm.engine.ops.op_fused_llm_attention", "fused_llm_attention", "rldx_backbone::fused_attention"),
    ("llm.engine.ops.op_fused_epilogue_add2_rmsnorm", "fused_epilogue_add2_rmsnorm",
     "rldx_backbone::fused_epilogue_add2_rmsnorm"),
    ("llm.engine.ops.op_fused_epilogue_add3_rmsnorm", "fused_epilogue_add3_rmsnorm",
     "rldx_backbone::fused_epilogue_add3_rmsnorm"),
    ("vision_encoder.engine.ops.op_fused_vision_attention", "vision_attention", "rldx_backbone::vision_attention"),
    ("memory.engine.ops.op_fused_memory_attention", "fused_memory_attention", "mem::fused_attention"),
    ("memory.engine.ops.op_fused_epilogue_add2_rmsnorm", "fused_epilogue_add2_rmsnorm",
     "mem::fused_epilogue_add2_rmsnorm"),
]


@pytest.mark.parametrize("module,name,qualname", OP_MODULES, ids=[q for _, _, q in OP_MODULES])
def test_op_modules_bind_the_rldx_amd_registrations(installed, module, name, qualname):
    op = getattr(sys.modules[module], name)
    assert op._qualname == qualname
    ns, _, opname = qualname.partition("::")
    assert getattr(getattr(torch.ops, ns), opname) is not None


def test_setup_helpers_closed_forms(installed):
    from llm.engine.kernels.fused_llm_attention import (prepare_fused_qkv_weight, prepare_norm_weight_rot,
                                                        prepare_signed_sin)
    from memory.engine.kernels.fused_memory_attention import prepare_rope_buffers

    g = torch.Generator().manual_seed(5)
    D = 8
    sin = torch.randn(3, D, generator=g).to(torch.bfloat16)
    s = prepare_signed_sin(sin, D)
    assert torch.equal(s[:, : D // 2], -sin[:, : D // 2]) and torch.equal(s[:, D // 2:], sin[:, D // 2:])
    w = torch.arange(D, dtype=torch.float32)
    assert prepare_norm_weight_rot(w, D).tolist() == [(d + D // 2) % D for d in range(D)]
    with pytest.raises(ValueError):
        prepare_signed_sin(sin, D + 2)

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj, self.k_proj, self.v_proj = (torch.nn.Linear(4, n, bias=False) for n in (6, 2, 2))

    layer = torch.nn.Module()
    layer.self_attn = Attn()
    fused = prepare_fused_qkv_weight(layer)
    a = layer.self_attn
    assert torch.equal(fused, torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).detach())

    class Rotary:  # the HF rotary-embedding call convention: (x, position_ids) -> cos, sin (1, M, D)
        dim = D

        def __call__(self, x, position_ids):
            ang = position_ids[0, :, None].float() * torch.arange(1, D + 1).float()
            return ang.cos()[None].to(x.dtype), ang.sin()[None].to(x.dtype)

    cos, ssin = prepare_rope_buffers(Rotary(), torch.arange(5)[None], "cpu")
    c_ref, s_ref = Rotary()(torch.empty(0, dtype=torch.bfloat16), torch.arange(5)[None])
    assert torch.equal(cos, c_ref[0]) and torch.equal(ssin, prepare_signed_sin(s_ref[0], D))


# ---------------------------------------------------------------------------
# model-level mirrors
# ---------------------------------------------------------------------------
@pytest.fixture
def model_installed():
    yield compat.install_model()
    compat.uninstall()


MODEL_SIGNATURES = [
    ("rldx.model.modules.norms", "create_norm_layer", [("norm_type", _EMPTY), ("dim", _EMPTY), ("eps", 1e-6)],
     "norms.py:25"),
    ("rldx.model.modules.norms", "create_qk_norm_layers", [("qk_norm", _EMPTY), ("head_dim", _EMPTY), ("eps", 1e-6)],
     "norms.py:44"),
    ("rldx.model.modules.action_model.ops", "precompute_freqs_cis",
     [("dim", _EMPTY), ("end", _EMPTY), ("theta", 10000.0)], "action_model/ops.py:11"),
    ("rldx.model.modules.action_model.ops", "apply_rotary_emb",
     [("xq", _EMPTY), ("xk", _EMPTY), ("freqs_cis", _EMPTY)], "action_model/ops.py:48-52"),
    ("rldx.model.modules.backbone.modeling_qwen3_vl", "apply_rotary_pos_emb",
     [("q", _EMPTY), ("k", _EMPTY), ("cos", _EMPTY), ("sin", _EMPTY), ("position_ids", None), ("unsqueeze_dim", 1)],
     "modeling_qwen3_vl.py:377"),
    ("rldx.model.modules.backbone.modeling_qwen3_vl", "rotate_half", [("x", _EMPTY)], "modeling_qwen3_vl.py:118"),
]


@pytest.mark.parametrize("module,fn,params,cite", MODEL_SIGNATURES, ids=[f for _, f, _, _ in MODEL_SIGNATURES])
def test_model_function_signatures(model_installed, module, fn, params, cite):
    f = getattr(sys.modules[module], fn)
    assert [(p.name, p.default) for p in inspect.signature(f).parameters.values()] == params, cite


def test_model_modules_match_reference_constructors_and_parameters(model_installed):
    """Constructor signatures and state-dict names, so reference checkpoints load
    (norms.py:13-16, action_model/ops.py:143-157)."""
    from rldx.model.modules.action_model.ops import SwiGLUFFN
    from rldx.model.modules.backbone.modeling_qwen3_vl import rotate_half
    from rldx.model.modules.norms import RMSNorm, create_norm_layer, create_qk_norm_layers

    assert [(p.name, p.default) for p in list(inspect.signature(RMSNorm.__init__).parameters.values())[1:]] == \
        [("dim", _EMPTY), ("eps", 1e-6)]
    assert [(p.name, p.default) for p in list(inspect.signature(SwiGLUFFN.__init__).parameters.values())[1:]] == \
        [("in_features", _EMPTY), ("hidden_features", None), ("out_features", None), ("act_layer", None),
         ("drop", 0.0), ("bias", True)]
    n = RMSNorm(64)
    assert list(n.state_dict()) == ["weight"] and n.weight.dtype == torch.float32 and torch.equal(n.weight, torch.ones(64))
    f = SwiGLUFFN(1536, 4096)
    assert {k: tuple(v.shape) for k, v in f.state_dict().items()} == {
        "w12.weight": (8192, 1536), "w12.bias": (8192,), "w3.weight": (1536, 4096), "w3.bias": (1536,)}
    assert list(SwiGLUFFN(128, 64, 32, bias=False).state_dict()) == ["w12.weight", "w3.weight"]
    assert isinstance(create_norm_layer("rms_norm", 64), RMSNorm)
    assert all(isinstance(m, torch.nn.Identity) for m in create_qk_norm_layers("none", 64))
    with pytest.raises(ValueError):
        create_norm_layer("batch_norm", 64)
    x = torch.arange(8.0).reshape(2, 4)
    assert torch.equal(rotate_half(x), torch.tensor([[-2.0, -3.0, 0.0, 1.0], [-6.0, -7.0, 4.0, 5.0]]))


def test_precompute_freqs_cis_closed_form(model_installed):
    """freqs[n][i] = exp(i n theta^(-2i/D)): unit modulus, angle n * theta^(-2i/D)."""
    from rldx.model.modules.action_model.ops import precompute_freqs_cis

    f = precompute_freqs_cis(8, 5, 100.0).to(torch.complex128)
    n = torch.arange(5, dtype=torch.float64)[:, None]
    ang = n * 100.0 ** (-torch.arange(0, 8, 2, dtype=torch.float64) / 8)
    assert f.shape == (5, 4) and torch.allclose(f.abs(), torch.ones(5, 4, dtype=torch.float64), atol=1e-6)
    assert torch.allclose(f, torch.polar(torch.ones_like(ang), ang), atol=1e-5)


def _write(root, rel, text):
    p = root / rel
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_text(text)


@pytest.fixture
def fake_reference(tmp_path, monkeypatch):
    """A reference tree on sys.path whose package __init__ files have side
    effects: rldx/__init__.py imports the model blocks (as rldx/__init__.py:66
    does), memory/engine/__init__.py imports its own ops module, which would
    register mem:: operators again (custom_memory_chain.py:18,25), and every
    executed module records itself in a list."""
    log = "import sys as _s\n_s.modules['_ref_log'].append(__name__)\n"
    _write(tmp_path, "rldx/__init__.py", log + "from .model.modules.action_model import blocks  # noqa\n")
    _write(tmp_path, "rldx/inference/__init__.py", log)
    _write(tmp_path, "rldx/inference/memory/__init__.py", log)
    _write(tmp_path, "rldx/inference/memory/engine/__init__.py",
           log + "import memory.engine.ops  # noqa\nraise RuntimeError('reference engine package ran')\n")
    _write(tmp_path, "rldx/inference/memory/engine/extra.py", log + "VALUE = 7\n")
    _write(tmp_path, "rldx/model/__init__.py", log)
    _write(tmp_path, "rldx/model/modules/__init__.py", log)
    _write(tmp_path, "rldx/model/modules/norms.py", log + "class RMSNorm: pass\n"
           "def create_norm_layer(*a, **k): return 'ref'\ndef create_qk_norm_layers(*a, **k): return 'ref'\n")
    _write(tmp_path, "rldx/model/modules/action_model/__init__.py", log)
    _write(tmp_path, "rldx/model/modules/action_model/ops.py", log + "class SwiGLUFFN: pass\n"
           "def apply_rotary_emb(*a): return 'ref'\ndef precompute_freqs_cis(*a, **k): return 'ref'\n")
    _write(tmp_path, "rldx/model/modules/action_model/blocks.py", log +
           "from .ops import SwiGLUFFN, apply_rotary_emb\nfrom ..norms import create_norm_layer, "
           "create_qk_norm_layers\n")
    monkeypatch.syspath_prepend(str(tmp_path))
    ran = []
    monkeypatch.setitem(sys.modules, "_ref_log", ran)
    before = set(sys.modules)
    yield ran
    compat.uninstall()
    for name in set(sys.modules) - before:
        if name == "rldx" or name.startswith("rldx.") or name.startswith("memory"):
            sys.modules.pop(name, None)


def test_install_runs_no_reference_package_init(fake_reference):
    """install() registers the mirrors without running any reference module:
    the fake engine package's __init__ (which re-imports its ops and raises)
    never runs, the mirrored ops module is ours under every alias, and a
    non-mirrored reference submodule stays importable through the stub
    package's __path__."""
    import importlib

    done = compat.install()
    assert fake_reference == [], f"reference modules ran: {fake_reference}"
    ours = done["memory.engine.ops"]
    assert ours.__name__.startswith("rldx_amd.compat.")
    assert sys.modules["rldx.inference.memory.engine.ops"] is ours
    extra = importlib.import_module("rldx.inference.memory.engine.extra")
    assert extra.VALUE == 7
    assert fake_reference == ["rldx.inference.memory.engine.extra"]


def test_install_model_rebinds_by_value_imports_and_restores(fake_reference):
    """install_model() replaces the norm / ops names in the reference modules
    and in every module that bound them by value (the fake blocks.py's
    `from .ops import SwiGLUFFN, ...`), and uninstall() restores the originals."""
    import importlib

    compat.install_model()
    blocks = importlib.import_module("rldx.model.modules.action_model.blocks")
    ref_ops = sys.modules["rldx.model.modules.action_model.ops"]
    from rldx_amd.compat.model.modules import norms as our_norms
    from rldx_amd.compat.model.modules.action_model import ops as our_ops

    assert blocks.SwiGLUFFN is our_ops.SwiGLUFFN and ref_ops.SwiGLUFFN is our_ops.SwiGLUFFN
    assert blocks.apply_rotary_emb is our_ops.apply_rotary_emb
    assert blocks.create_norm_layer is our_norms.create_norm_layer
    assert blocks.create_qk_norm_layers is our_norms.create_qk_norm_layers
    compat.uninstall()
    assert blocks.SwiGLUFFN is ref_ops.SwiGLUFFN and blocks.SwiGLUFFN.__module__ == ref_ops.__name__
    assert blocks.apply_rotary_emb() == "ref" and blocks.create_norm_layer() == "ref"
