"""Sluice plugin entry point (vLLM ``general_plugins``), MI355X build.

Mirrors src/sluice/plugin.py:27-96: ``register()`` is a no-op unless
``SLUICE_SLOTS`` parses to a positive int (an invalid value warns and does
nothing), refuses vLLM's V2 model runner, then patches vLLM's
``create_offloader`` factory (at its definition and in the model-runner
module that imported it) so the active offloader is this package's
``ExpertStreamOffloader``, and wraps ``GPUModelRunner.load_model`` to call
``attach_model`` on the loaded model.  vLLM is optional here: without it the
function validates the environment and returns, and the offloader can be
driven directly (``sluice_amd.decoder`` does so).
"""

import logging
import os

logger = logging.getLogger("sluice")

SLOTS_ENV = "SLUICE_SLOTS"

# The live offloader instance for this process (set by the patched factory).
_ACTIVE = None


def slots_from_env():
    """The SLUICE_SLOTS value, or None when unset/invalid (with a warning)."""
    raw = os.environ.get(SLOTS_ENV)
    if not raw:
        return None
    try:
        slots = int(raw)
        assert slots > 0
    except (ValueError, AssertionError):
        logger.warning("Sluice: ignoring invalid %s=%r (want a positive int).", SLOTS_ENV, raw)
        return None
    return slots


def register() -> None:
    """vLLM ``general_plugins`` hook.  No-op unless ``SLUICE_SLOTS`` is set."""
    slots = slots_from_env()
    if slots is None:
        return

    try:
        import vllm.envs as vllm_envs

        if getattr(vllm_envs, "VLLM_USE_V2_MODEL_RUNNER", False):
            raise RuntimeError(
                "Sluice requires the V1 model runner but VLLM_USE_V2_MODEL_RUNNER is set — the "
                "V2 runner never invokes create_offloader/post_init, so Sluice (and its "
                "correctness guards) would silently not run. Unset VLLM_USE_V2_MODEL_RUNNER.")
    except ImportError:
        logger.info("Sluice: vLLM not importable; %s=%d recorded, nothing to patch.", SLOTS_ENV,
                    slots)
        return

    import vllm.model_executor.offloader.base as base_mod

    from sluice_amd.offloader import ExpertStreamOffloader

    def _create_offloader(offload_config):  # noqa: ANN001
        global _ACTIVE
        _ACTIVE = ExpertStreamOffloader(expert_cache_slots=slots)
        return _ACTIVE

    base_mod.create_offloader = _create_offloader
    try:
        import vllm.v1.worker.gpu_model_runner as gmr

        if hasattr(gmr, "create_offloader"):
            gmr.create_offloader = _create_offloader
        _orig_load = gmr.GPUModelRunner.load_model

        def load_model(self, *a, **k):  # noqa: ANN001
            out = _orig_load(self, *a, **k)
            try:
                mdl = getattr(self, "model", None)
                if _ACTIVE is not None and mdl is not None:
                    _ACTIVE.attach_model(mdl)
            except Exception:
                logger.exception("Sluice: attach_model failed (router-split not armed).")
            return out

        gmr.GPUModelRunner.load_model = load_model
    except Exception:  # pragma: no cover - depends on the vLLM version present
        logger.debug("Sluice: gpu_model_runner not patchable; relying on base.")

    logger.info("Sluice: activated via %s=%d (expert offloading on).", SLOTS_ENV, slots)
