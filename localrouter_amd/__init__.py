"""localrouter_amd -- an MI355X-native (gfx950) implementation of LocalRouter's DiT joint-attention hot path.

The product is liblr_attn.so: hand-written CDNA4 HIP kernels (csrc/) behind the C ABI of include/lr_attn.h.
This package adds the ctypes binding (_lib), a torch-facing mirror of the reference engine's kernel bindings (ops),
and the host RoPE table builders (rope). There is no CPU fallback: without the built library every op raises.
"""
from . import rope  # noqa: F401  (numpy only)

__all__ = ["rope", "ops", "build"]


def __getattr__(name):
    # `ops` imports torch: load it on first use only
    if name == "ops":
        import importlib
        return importlib.import_module(".ops", __name__)
    raise AttributeError(name)
