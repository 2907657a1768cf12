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
names).  Parent packages that are not imported yet are registered as stub
packages whose __path__ is the reference's directory (found without importing
anything), so the reference's package __init__ files -- some of which import
their Triton ops -- never run, while its other submodules stay importable.
Call it before importing the reference's chains.

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
  action_model/engine/custom_action_model_chain.py               CustomActionHeadChain, build_/compile_custom_action_model_chain
  action_model/engine/custom_expanded_action_model_chain.py      CustomExpandedActionHeadChain,
                                                                 build_/compile_custom_expanded_action_model_chain
and the op registration modules (engine/ops/__init__.py and op_*.py) of the
same directories.  Not mirrored: the Triton kernel objects the reference's
op modules launch directly (rmsnorm_rope_kernel*, the dormant
attention_fusion_* alternatives) and the vision MLP / LayerNorm operators,
which have no rldx_amd kernel.
"""

from __future__ import annotations

import importlib
import importlib.machinery
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
    """Make the parent packages of `name` importable without running any of the
    reference's code: a package already in sys.modules is kept; any other is
    registered as a stub package whose __path__ lists the reference's directory
    for it when the reference is on sys.path (located with PathFinder, which
    imports nothing), else an empty __path__ (so that `import
    double_stream.engine.ops` also works without the reference installed).
    The reference's package __init__ never runs: it may import the reference's
    own Triton ops (e.g. memory/engine/__init__.py)."""
    parts = name.split(".")[:-1]
    for i in range(1, len(parts) + 1):
        pkg = ".".join(parts[:i])
        if pkg in sys.modules:
            continue
        parent = sys.modules[".".join(parts[:i - 1])] if i > 1 else None
        search = list(getattr(parent, "__path__", None) or []) if parent is not None else None
        try:
            spec = importlib.machinery.PathFinder.find_spec(pkg, search)
        except (ImportError, ValueError):
            spec = None
        locs = list(spec.submodule_search_locations or []) if spec is not None else []
        mod = types.ModuleType(pkg, "stub package of mirrored reference modules (its __init__ is not run)")
        mod.__path__ = locs
        mod.__spec__ = importlib.machinery.ModuleSpec(pkg, None, is_package=True)
        mod.__spec__.submodule_search_locations = locs
        sys.modules[pkg] = mod
        _added.append(pkg)
        if parent is not None:
            setattr(parent, parts[i - 1], mod)


_added: list = []  # sys.modules names install() registered or created
_rebound: list = []  # (module, attribute, original value) install_model() replaced


def install() -> dict:
    """Register the mirrored modules under the reference's module names, before
    any module of the reference is imported.  Returns {reference name: module}."""
    done = {}
    mirrors = [(path, importlib.import_module(_PKG + "." + path)) for path in modules()]  # ours only
    for path, mod in mirrors:
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


_MISSING = object()


def _rebind(module, attr: str, value) -> None:
    _rebound.append((module, attr, getattr(module, attr, _MISSING)))
    setattr(module, attr, value)


def install_model() -> dict:
    """Model-level drop-in: RMSNorm / create_norm_layer / create_qk_norm_layers
    (rldx/model/modules/norms.py), precompute_freqs_cis / apply_rotary_emb /
    SwiGLUFFN (action_model/ops.py), rotate_half / apply_rotary_pos_emb
    (backbone/modeling_qwen3_vl.py).  Where the reference module imports, its
    attributes of those names are replaced, and so is every binding of the
    original objects in any loaded module (the reference's blocks.py binds
    SwiGLUFFN, apply_rotary_emb, create_norm_layer and create_qk_norm_layers by
    value with `from ... import`, blocks.py:10-16, and importing the norms
    module first runs rldx/__init__.py, which imports the blocks); uninstall()
    restores every original.  Models built before the call keep the layers they
    were built with.  Where the reference does not import, the mirror is
    registered under its name.  Returns {reference name: module}."""
    done = {}
    for ref_name, ours in _MODEL.items():
        mod = importlib.import_module(ours)
        try:
            ref = importlib.import_module(ref_name)
        except ImportError:
            ref = None
        if ref is not None and ref is not mod:
            originals = {attr: getattr(ref, attr) for attr in mod.__all__ if hasattr(ref, attr)}
            for attr in mod.__all__:
                _rebind(ref, attr, getattr(mod, attr))
            for other in list(sys.modules.values()):  # by-value bindings elsewhere
                if other is None or other is ref or other is mod:
                    continue
                for attr, orig in originals.items():
                    if getattr(other, attr, None) is orig:
                        _rebind(other, attr, getattr(mod, attr))
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
    """Remove what install() / install_model() registered and restore every
    attribute install_model() replaced (the operators stay registered)."""
    while _rebound:
        module, attr, orig = _rebound.pop()
        if orig is _MISSING:
            delattr(module, attr)
        else:
            setattr(module, attr, orig)
    while _added:
        sys.modules.pop(_added.pop(), None)
