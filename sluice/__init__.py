"""Sluice: routing-aware MoE expert offloading for vLLM, MI355X build.

The reference package's import surface (src/sluice/__init__.py:4-7):
``ExpertStreamOffloader`` and ``__version__``, and the ``sluice.plugin``
module its vLLM entry point names.  The implementation lives in
``sluice_amd`` (HIP kernels for gfx950 behind a C ABI).
"""

from sluice_amd import __version__

__all__ = ["ExpertStreamOffloader", "__version__"]


def __getattr__(name):
    # importing the package (vLLM loads sluice.plugin in every process) must
    # not load torch or the native library
    if name == "ExpertStreamOffloader":
        from sluice_amd.offloader import ExpertStreamOffloader

        return ExpertStreamOffloader
    raise AttributeError(name)
