"""MI355X-native (gfx950) fused Matmul -> row-Softmax, the hot path of the
Welder typical chain, behind the reference's compile / solver C entry points.

Importing the package needs neither a GPU nor the built library; the first
call into the kernels loads ``libwtc_hip.so`` and fails loudly if it is
missing.
"""
from . import _lib  # noqa: F401

__all__ = ["matmul_softmax", "workspace_size", "new_workspace", "read_error_flags"]


def __getattr__(name):
    if name in __all__:
        from . import chain
        return getattr(chain, name)
    raise AttributeError(name)
