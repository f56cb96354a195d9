"""Opt-in vLLM general plugin (the vllm.general_plugins entry point; the role
of npu_sparse_attn_sharedkv_int8/vllm_plugin.py in the reference checkout).

SHAREDKV_INT8_MODE selects what register() does; unset, vLLM runs unchanged:
  calibrate   every cache write of the bound attention class is observed by a
              calibration.CacheObserver writing to SHAREDKV_CALIBRATION_DIR,
              then proceeds in BF16 (the offline step that produces scales)
  int8        vllm_adapter.install(): cache writes and sparse attention run on
              the HIP kernels with the frozen scales of SHAREDKV_SCALES
The engine classes to hook come from an EngineBinding: passed to register()
by a deployment, or named in SHAREDKV_VLLM_TARGETS as JSON
{"impl": "module:Class", "cache_specs": ["module:Class", ...],
 "compact_pages": false}.  (vLLM-ROCm does not fix the names of its
DeepSeek-V4 attention classes, so the deployment names them.)
"""
import importlib
import json
import os

from .vllm_adapter import EngineBinding, describe_dsa_impl

MODES = ("calibrate", "int8")
TARGETS_ENV = "SHAREDKV_VLLM_TARGETS"


class _State:
    mode = None          # the mode register() installed, or None
    observer = None      # the CacheObserver of calibrate mode


state = _State()


def resolve(name):
    """'package.module:Outer.Inner' -> the named object."""
    module, sep, qualified = name.partition(":")
    if not sep or not module or not qualified:
        raise ValueError(f"Expected 'module:Qualified.Name', got {name!r}")
    target = importlib.import_module(module)
    for attribute in qualified.split("."):
        target = getattr(target, attribute)
    return target


def binding_from_env():
    text = os.environ.get(TARGETS_ENV)
    if not text:
        raise RuntimeError(f"{TARGETS_ENV} must name the engine's DeepSeek-V4 sparse attention class "
                           "(and its cache-spec classes)")
    spec = json.loads(text)
    return EngineBinding(impl=resolve(spec["impl"]), cache_specs=tuple(resolve(n) for n in spec.get("cache_specs", ())),
                         compact_pages=bool(spec.get("compact_pages", os.environ.get("SHAREDKV_COMPACT_PAGES") == "1")))


def observe_writes(binding, observer):
    """Wrap the binding's cache-write method: observe, then write in BF16."""
    bf16_write = getattr(binding.impl, binding.write_method)

    def write(self, cache, kv, slot_mapping, *, quantize):
        layer = binding.describe(self)
        if layer.quantized_elsewhere:
            raise ValueError("Shared-KV calibration requires the ordinary BF16 DSA path")
        observer.observe(layer.prefix, "cmp" if quantize else "ori", cache, kv, slot_mapping)
        return bf16_write(self, cache, kv, slot_mapping, quantize=quantize)

    setattr(binding.impl, binding.write_method, write)


def register(binding=None):
    """Install the mode SHAREDKV_INT8_MODE names (once per process)."""
    mode = os.environ.get("SHAREDKV_INT8_MODE", "")
    if not mode or state.mode is not None:
        return
    if mode not in MODES:
        raise ValueError(f"Unsupported SHAREDKV_INT8_MODE={mode!r}")
    directory = os.environ.get("SHAREDKV_CALIBRATION_DIR")
    if mode == "calibrate" and not directory:
        raise ValueError("calibrate mode requires SHAREDKV_CALIBRATION_DIR")
    binding = binding if binding is not None else binding_from_env()
    if mode == "calibrate":
        from .calibration import CacheObserver
        state.observer = CacheObserver(directory)
        observe_writes(binding, state.observer)
    else:
        from .vllm_adapter import install
        install(binding)
    state.mode = mode


__all__ = ["EngineBinding", "binding_from_env", "describe_dsa_impl", "observe_writes", "register", "resolve", "state"]
