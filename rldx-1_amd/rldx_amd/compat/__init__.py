"""Drop-in mirror of the reference's inference launcher and operator modules.

The reference's chains import their kernels by module name, with the
inference directories on sys.path (rldx/inference/__init__.py:13-37):

    from double_stream.engine.kernels.vl_epilogue_ln import fused_vl_epilogue_ln
    from llm.engine.kernels.fused_llm_attention import prepare_signed_sin, ...
    import double_stream.engine.ops           # registers ds:: operators

`compat/inference/` mirrors those modules file for file (same module names,
function names, signatures and defaults), backed by the gfx950 kernels of
librldx_amd.so.  `install()` registers every mirrored module in sys.modules
under the names the reference imports it by -- the fully qualified
`rldx.inference.<path>`, the path below rldx/inference, and the path below
its first directory (`double_stream.engine...`, `llm.engine...`) -- so a chain
imported afterwards binds the MI355X launchers, and the reference's Triton op
registrations are never imported (the rldx_amd registrations take their
names).  Call it before importing the reference's chains.

Mirrored launchers (reference file: function):
  action_model/double_stream/engine/kernels/vl_epilogue_ln.py    fused_vl_epilogue_ln
  action_model/double_stream/engine/kernels/grouped_res_ln.py    fused_grouped_res_ln
  action_model/double_stream/engine/kernels/grouped_swiglu.py    fused_grouped_swiglu
  action_model/single_stream/engine/kernels/ss_epilogue_ln.py    fused_ss_epilogue_ln
  action_model/single_stream/engine/kernels/fused_mlp_swiglu.py  fused_mlp_swiglu
  backbone/llm/engine/kernels/fused_llm_attention.py             forward, prepare_signed_sin,
                                                                 prepare_norm_weight_rot, prepare_fused_qkv_weight,
                                                                 autotune_split_m_threshold
  backbone/llm/engine/kernels/fused_add2_rmsnorm.py, fused_add3_rmsnorm.py   forward
  backbone/vision_encoder/engine/kernels/fused_vision_attention.py           forward, autotune_split_m_threshold
  memory/engine/kernels/fused_memory_attention.py                forward, prepare_signed_sin, prepare_rope_buffers,
                                                                 prepare_fused_qkv_weight
  memory/engine/kernels/fused_add2_rmsnorm.py                    forward
and the op registration modules (engine/ops/__init__.py and op_*.py) of the
same directories.  Not mirrored: the Triton kernel objects the reference's
op modules launch directly (rmsnorm_rope_kernel*, the dormant
attention_fusion_* alternatives) and the vision MLP / LayerNorm operators,
which have no rldx_amd kernel.
"""

from __future__ import annotations

import importlib
import importlib.util
import sys
import types
from pathlib import Path

_ROOT = Path(__file__).resolve().parent / "inference"
_PKG = __name__ + ".inference"
# first directories below rldx/inference whose children the reference also
# imports as top-level modules (its sys.path roots)
_SUB_ROOTS = ("action_model", "backbone")


def modules() -> list:
    """Mirrored module paths below rldx/inference, dotted ('backbone.llm.engine.kernels.fused_add2_rmsnorm')."""
    out = []
    for p in sorted(_ROOT.rglob("*.py")):
        rel = p.relative_to(_ROOT).with_suffix("")
        parts = list(rel.parts)
        if parts[-1] == "__init__":
            parts = parts[:-1]
        if parts:
            out.append(".".join(parts))
    return out


def aliases(path: str) -> list:
    """The module names the reference imports mirrored module `path` by."""
    names = ["rldx.inference." + path, path]
    first, _, rest = path.partition(".")
    if first in _SUB_ROOTS and rest:
        names.append(rest)
    return names


def _parent_packages(name: str) -> None:
    """Make the parent packages of `name` importable: from the reference when it
    is on sys.path (its own package modules, imported as usual), else as empty
    package modules (so that `import double_stream.engine.ops` also works
    without the reference installed)."""
    parts = name.split(".")[:-1]
    for i in range(1, len(parts) + 1):
        pkg = ".".join(parts[:i])
        if pkg in sys.modules:
            continue
        try:
            spec = importlib.util.find_spec(pkg)
        except (ImportError, ValueError):
            spec = None
        if spec is not None:
            importlib.import_module(pkg)
            continue
        mod = types.ModuleType(pkg, "package of mirrored reference modules (the reference is not installed)")
        mod.__path__ = []
        sys.modules[pkg] = mod
        _added.append(pkg)
        if i > 1:
            setattr(sys.modules[".".join(parts[:i - 1])], parts[i - 1], mod)


_added: list = []  # sys.modules names install() registered or created


def install() -> dict:
    """Register the mirrored modules under the reference's module names.
    Returns {reference name: module}."""
    done = {}
    for path in modules():
        mod = importlib.import_module(_PKG + "." + path)
        for name in aliases(path):
            if name not in done:
                _parent_packages(name)
            if sys.modules.get(name) is not mod:
                _added.append(name)
            sys.modules[name] = mod
            done[name] = mod
            parent, _, leaf = name.rpartition(".")
            setattr(sys.modules[parent], leaf, mod)
    return done


# model-level mirrors: reference module -> mirror module
_MODEL = {
    "rldx.model.modules.norms": __name__ + ".model.modules.norms",
    "rldx.model.modules.action_model.ops": __name__ + ".model.modules.action_model.ops",
    "rldx.model.modules.backbone.modeling_qwen3_vl": __name__ + ".model.modules.backbone.modeling_qwen3_vl",
}


def install_model() -> dict:
    """Model-level drop-in: RMSNorm / create_norm_layer / create_qk_norm_layers
    (rldx/model/modules/norms.py), precompute_freqs_cis / apply_rotary_emb /
    SwiGLUFFN (action_model/ops.py), rotate_half / apply_rotary_pos_emb
    (backbone/modeling_qwen3_vl.py).  Where the reference module imports, its
    attributes of those names are replaced (call this before the model is
    built: its blocks bind the names at construction); where it does not, the
    mirror is registered under its name.  Returns {reference name: module}."""
    done = {}
    for ref_name, ours in _MODEL.items():
        mod = importlib.import_module(ours)
        try:
            ref = importlib.import_module(ref_name)
        except ImportError:
            ref = None
        if ref is not None and ref is not mod:
            for attr in mod.__all__:
                setattr(ref, attr, getattr(mod, attr))
            done[ref_name] = ref
            continue
        _parent_packages(ref_name)
        if sys.modules.get(ref_name) is not mod:
            _added.append(ref_name)
        sys.modules[ref_name] = mod
        parent, _, leaf = ref_name.rpartition(".")
        setattr(sys.modules[parent], leaf, mod)
        done[ref_name] = mod
    return done


def uninstall() -> None:
    """Remove what install() registered (the operators stay registered)."""
    while _added:
        sys.modules.pop(_added.pop(), None)
