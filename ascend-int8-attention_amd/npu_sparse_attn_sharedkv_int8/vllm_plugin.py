"""Opt-in vLLM general plugin: SHAREDKV_INT8_MODE unset leaves vLLM unchanged.

Interface counterpart: npu_sparse_attn_sharedkv_int8/vllm_plugin.py:1-67 of
the reference checkout.  Modes, as there:
  calibrate   observe every cache write (calibration.CacheObserver under
              SHAREDKV_CALIBRATION_DIR) and let the BF16 write proceed
  int8        route cache writes and sparse attention to the HIP kernels
              (vllm_adapter.install) with the frozen scales of SHAREDKV_SCALES

The reference patches vllm_ascend's DeepSeek-V4 classes by name.  The
classes of a vLLM-ROCm deployment are named by the deployment instead, in
SHAREDKV_VLLM_TARGETS, a JSON object of "module:Qualified.Name" strings:
  impl              attention implementation (get_kv_plan, _write_kv_cache)
  cache_specs       list of classes with get_kv_cache_spec(config)
  metadata_builder  builder whose _build_sas_metadata sees max_seqlen_kv
  draft_model       optional model with _store_standard_swa_kv (draft context
                    KV written outside the attention layer)
or handed to register(targets=...) directly.
"""
import importlib
import json
import logging
import os

_registered = False
_observer = None
TARGETS_ENV = "SHAREDKV_VLLM_TARGETS"


def layer_prefix(impl):
    return impl.swa_cache_layer.prefix.removesuffix(".swa_cache")


def resolve(name):
    """'package.module:Outer.Inner' -> the object."""
    module, _, qualified = name.partition(":")
    if not module or not qualified:
        raise ValueError(f"Expected 'module:Qualified.Name', got {name!r}")
    obj = importlib.import_module(module)
    for part in qualified.split("."):
        obj = getattr(obj, part)
    return obj


def targets_from_env():
    text = os.environ.get(TARGETS_ENV)
    if not text:
        raise RuntimeError(f"{TARGETS_ENV} must name the engine's DeepSeek-V4 attention classes "
                           "(impl, cache_specs, metadata_builder[, draft_model])")
    names = json.loads(text)
    return {"impl": resolve(names["impl"]),
            "cache_specs": [resolve(n) for n in names.get("cache_specs", ())],
            "metadata_builder": resolve(names["metadata_builder"]) if names.get("metadata_builder") else None,
            "draft_model": resolve(names["draft_model"]) if names.get("draft_model") else None}


def register(targets=None):
    global _registered, _observer
    if os.environ.get("SHAREDKV_PROFILE_DIAGNOSTICS_DIR"):
        logging.getLogger("vllm.sharedkv_c8").warning(
            "SHAREDKV_PROFILE_DIAGNOSTICS_DIR is ignored: serving diagnostics are not part of this build")
    mode = os.environ.get("SHAREDKV_INT8_MODE", "")
    if not mode or _registered:
        return
    if mode not in ("calibrate", "int8"):
        raise ValueError(f"Unsupported SHAREDKV_INT8_MODE={mode!r}")
    directory = os.environ.get("SHAREDKV_CALIBRATION_DIR")
    if mode == "calibrate" and not directory:
        raise ValueError("calibrate mode requires SHAREDKV_CALIBRATION_DIR")
    targets = targets if targets is not None else targets_from_env()
    impl_cls = targets["impl"]

    if mode == "calibrate":
        from .calibration import CacheObserver
        _observer = CacheObserver(directory)
        original_write = impl_cls._write_kv_cache

        def observed_write(self, cache, kv, slot_mapping, *, quantize):
            if getattr(self, "turboquant", None) is not None:
                raise ValueError("Shared-KV calibration requires the ordinary BF16 DSA path")
            _observer.observe(layer_prefix(self), "cmp" if quantize else "ori", cache, kv, slot_mapping)
            return original_write(self, cache, kv, slot_mapping, quantize=quantize)

        impl_cls._write_kv_cache = observed_write
    else:
        from .vllm_adapter import install
        install(impl_cls, targets.get("cache_specs", ()), targets.get("metadata_builder"))

    draft = targets.get("draft_model")
    if draft is not None:
        # Draft-context KV is written outside the attention layer; send it
        # through the same (observed or INT8) original-cache writer.
        def store_draft_context(self, shared_kv, slot_mapping, attn=None):
            if slot_mapping is None or slot_mapping.numel() == 0:
                return
            if attn is None:
                raise ValueError("Draft context writes need the attention layer")
            layer = attn.dsa_attn.swa_cache_layer
            cache = getattr(layer, "kv_cache", None)
            if cache is None:
                return
            while isinstance(cache, (tuple, list)) and len(cache) == 1:
                cache = cache[0]
            impl = attn.dsa_attn.dsa_attn.impl
            if slot_mapping.ndim == 1:
                slot_mapping = impl.get_kv_plan().format_dsa_slot_mapping(slot_mapping, layer.block_size)
            impl._write_kv_cache(cache, shared_kv, slot_mapping, quantize=False)

        draft._store_standard_swa_kv = store_draft_context
    _registered = True
