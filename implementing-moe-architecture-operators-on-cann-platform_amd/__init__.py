"""MI355X-native (gfx950) MoE layer: MoeRoutingTopK -> MoeExpertFFN -> MoeCombine.

The operators run as hand-written HIP kernels in libmoe_mi355x.so behind the C ABI of include/moe_ops.h.
`_lib` is the ctypes binding of that ABI, `ops` the torch-tensor mirror of the reference's operators,
`torch_ops` their torch.library registration (torch.ops.moe_mi355x.*), `synth` the synthetic-input generator,
`build` the in-tree build of the library.
"""
from __future__ import annotations

from . import _lib, synth
from ._lib import MoeError

__all__ = ["MoeError", "_lib", "synth", "ops", "torch_ops", "load_library"]


def load_library():
    """Load libmoe_mi355x.so (raises RuntimeError if it has not been built)."""
    return _lib.load()


def __getattr__(name):
    if name in ("ops", "torch_ops"):  # torch is imported only when the tensor-level API is used
        import importlib

        mod = importlib.import_module(f"{__name__}.{name}")
        globals()[name] = mod
        return mod
    raise AttributeError(name)
