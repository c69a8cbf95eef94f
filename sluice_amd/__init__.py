"""Sluice on MI355X: routing-aware MoE expert offloading, routed-MoE decode
hot path (top-k routing, streaming gap, grouped SwiGLU expert product over
slot buffers, weighted combine) on hand-written gfx950 HIP kernels."""

__version__ = "0.1.0"


def __getattr__(name):
    # Lazy: importing the package (e.g. for plugin.register) must not pull in
    # torch or the native library.
    if name == "ExpertStreamOffloader":
        from sluice_amd.offloader import ExpertStreamOffloader

        return ExpertStreamOffloader
    raise AttributeError(name)


__all__ = ["ExpertStreamOffloader", "__version__"]
