"""vLLM ``general_plugins`` hook of the MI355X build.

The entry point is ``sluice = "sluice.plugin:register"`` (the reference's
pyproject.toml:34-35); ``sluice.plugin`` re-exports ``register`` from here.
What it does is the reference's contract (src/sluice/plugin.py:27-96):

  * nothing unless ``SLUICE_SLOTS`` holds a positive int (anything else is
    ignored with a warning);
  * refuse vLLM's V2 model runner, which never calls the offloader
    lifecycle;
  * make vLLM's ``create_offloader`` factory return this package's
    ``ExpertStreamOffloader`` -- at its definition and in the model runner
    module that imported it by name;
  * after ``GPUModelRunner.load_model``, hand the loaded model to the
    offloader's ``attach_model`` (which arms the router-split entries).

Without vLLM the hook only validates the environment; the offloader can
then be driven directly (``sluice_amd.decoder`` does so).
"""

import logging
import os
from typing import Optional

logger = logging.getLogger("sluice")

SLOTS_ENV = "SLUICE_SLOTS"

# The offloader the patched factory made last in this process.
_ACTIVE = None


def slots_from_env() -> Optional[int]:
    """The SLUICE_SLOTS value, or None when unset or not a positive int."""
    raw = os.environ.get(SLOTS_ENV)
    if not raw:
        return None
    try:
        slots = int(raw)
    except ValueError:
        slots = 0
    if slots <= 0:
        logger.warning("Sluice: ignoring invalid %s=%r (want a positive int).", SLOTS_ENV, raw)
        return None
    return slots


class _Activation:
    """The patches register() installs for one SLUICE_SLOTS value."""

    def __init__(self, slots: int):
        self.slots = slots

    def create_offloader(self, offload_config=None):  # noqa: ARG002 - vLLM's factory signature
        global _ACTIVE
        from sluice_amd.offloader import ExpertStreamOffloader

        _ACTIVE = ExpertStreamOffloader(expert_cache_slots=self.slots)
        return _ACTIVE

    @staticmethod
    def attach_after(load_model):
        """GPUModelRunner.load_model, then attach_model on the loaded model
        (a failure there leaves the stock MoE path and is logged)."""

        def load_model_then_attach(runner, *args, **kwargs):
            result = load_model(runner, *args, **kwargs)
            model = getattr(runner, "model", None)
            if _ACTIVE is not None and model is not None:
                try:
                    _ACTIVE.attach_model(model)
                except Exception:  # noqa: BLE001
                    logger.exception("Sluice: attach_model failed; MoE layers run the stock "
                                     "path (router-split not armed).")
            return result

        load_model_then_attach.__wrapped__ = load_model
        return load_model_then_attach


def _refuse_v2_runner() -> None:
    try:
        import vllm.envs as vllm_envs  # type: ignore
    except ImportError:
        return
    if getattr(vllm_envs, "VLLM_USE_V2_MODEL_RUNNER", False):
        raise RuntimeError(
            "Sluice needs vLLM's V1 model runner: with VLLM_USE_V2_MODEL_RUNNER set, "
            "create_offloader and post_init are never called, so the expert cache would not be "
            "installed and its checks would not run. Unset VLLM_USE_V2_MODEL_RUNNER.")


def register() -> None:
    """vLLM ``general_plugins`` hook.  No-op unless ``SLUICE_SLOTS`` is set."""
    slots = slots_from_env()
    if slots is None:
        return
    _refuse_v2_runner()
    try:
        import vllm.model_executor.offloader.base as base_mod  # type: ignore
    except ImportError:
        logger.info("Sluice: %s=%d set but vLLM is not importable; nothing to patch.",
                    SLOTS_ENV, slots)
        return
    act = _Activation(slots)
    factory = act.create_offloader  # one object, installed everywhere
    base_mod.create_offloader = factory
    try:
        import vllm.v1.worker.gpu_model_runner as gmr  # type: ignore
    except Exception:  # noqa: BLE001 - another vLLM layout: the base patch alone
        logger.debug("Sluice: vLLM's gpu_model_runner not importable; patched the base factory.")
    else:
        if hasattr(gmr, "create_offloader"):
            gmr.create_offloader = factory
        runner_cls = getattr(gmr, "GPUModelRunner", None)
        if runner_cls is not None and hasattr(runner_cls, "load_model"):
            runner_cls.load_model = act.attach_after(runner_cls.load_model)
    logger.info("Sluice: %s=%d, expert offloading on.", SLOTS_ENV, slots)
