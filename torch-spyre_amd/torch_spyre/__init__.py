"""torch_spyre: the "spyre" PrivateUse1 device of PyTorch, backed by MI355X.

Drop-in for the reference package of the same name (torch_spyre/__init__.py
in the torch-spyre tree): the same autoload entry point, device name,
`torch.spyre` module functions and lazy native initialisation.  Device memory
is MI355X HBM, eager ops run hand-written gfx950 HIP kernels through the C-ABI
library (include/spyre_hip.h) and torch.compile lowers to the same kernels.

Differences from the reference, on purpose:
  * device_count() is the number of visible GPUs, not a constant 1;
  * a child started by a Python parent is NOT locked out of the device (the
    reference marks it "bad fork" via psutil, __init__.py:30-45); only a
    forked child of an initialised parent is, as with torch.cuda.
"""

from __future__ import annotations

import importlib
import os
import threading
import types

from .constants import DEVICE_NAME
from ._monkey_patch import _patch_tensor_for_spyre

_runtime_init_lock = threading.Lock()


class _SpyreImpl:
    """State behind the `torch.spyre` module (reference: _SpyreImpl,
    torch_spyre/__init__.py:25-101)."""

    def __init__(self):
        self._initialized = False
        self._in_bad_fork = False
        try:
            os.register_at_fork(after_in_child=self._mark_after_fork)
        except Exception:  # pragma: no cover - platform without fork hooks
            pass

    def __getattr__(self, name):
        if name.startswith("__") or name in ("_C",):
            if name == "_C":
                self._lazy_init()
                return super().__getattribute__(name)
            raise AttributeError(name)
        self._lazy_init()
        return super().__getattribute__(name)

    def _lazy_init(self):
        if self._initialized:
            return
        if self._in_bad_fork:
            raise RuntimeError(
                "torch.spyre: cannot re-initialise the device in a forked child process; "
                "use the 'spawn' start method")
        with _runtime_init_lock:
            if self._initialized:
                return
            self._C = importlib.import_module("torch_spyre._C")
            self._C.start_runtime()
            self._initialized = True

    def _is_in_bad_fork(self) -> bool:
        return self._in_bad_fork

    def _mark_after_fork(self):
        if self._initialized:
            self._in_bad_fork = True
            self._initialized = False

    def is_initialized(self) -> bool:
        return self._initialized

    def manual_seed(self, seed: int, device: int | None = None) -> None:
        self._lazy_init()
        self._C.manual_seed(int(seed), -1 if device is None else int(device))

    def manual_seed_all(self, seed: int) -> None:
        self._lazy_init()
        self._C.manual_seed_all(int(seed))

    def is_available(self) -> bool:
        try:
            self._lazy_init()
        except Exception:
            return False
        return self._C.device_count() > 0

    def device_count(self) -> int:
        try:
            self._lazy_init()
        except Exception:
            return 0
        return int(self._C.device_count())

    def current_device(self) -> int:
        self._lazy_init()
        return int(self._C.current_device())

    def set_device(self, idx) -> None:
        self._lazy_init()
        if hasattr(idx, "index"):
            idx = 0 if idx.index is None else idx.index
        self._C.set_device(int(idx))

    def synchronize(self, device=None) -> None:
        self._lazy_init()
        self._C.synchronize(-1 if device is None else int(getattr(device, "index", device) or 0))


def make_spyre_module() -> types.ModuleType:
    """Module object registered as `torch.spyre` (reference:
    make_spyre_module, torch_spyre/__init__.py:104-137)."""
    impl = _SpyreImpl()
    mod = types.ModuleType(DEVICE_NAME)
    mod.__doc__ = "Spyre backend module (MI355X HIP implementation)."
    mod._is_in_bad_fork = impl._is_in_bad_fork
    mod.manual_seed = impl.manual_seed
    mod.manual_seed_all = impl.manual_seed_all
    mod.is_available = impl.is_available
    mod.device_count = impl.device_count
    mod.current_device = impl.current_device
    mod.set_device = impl.set_device
    mod.synchronize = impl.synchronize
    mod.is_initialized = impl.is_initialized
    mod.memory_allocated = lambda device=None: impl._C.memory_allocated(
        -1 if device is None else int(getattr(device, "index", device) or 0))
    mod.memory_reserved = lambda device=None: impl._C.memory_reserved(
        -1 if device is None else int(getattr(device, "index", device) or 0))
    mod.max_memory_allocated = lambda device=None: impl._C.max_memory_allocated(
        -1 if device is None else int(getattr(device, "index", device) or 0))
    mod.empty_cache = lambda: impl._C.empty_cache()
    mod._lazy_init = impl._lazy_init
    mod._is_compiled = lambda: True

    from . import graphs as _graphs

    mod.SpyreGraph = _graphs.SpyreGraph
    mod.graph = _graphs.graph

    def __getattr__(name):
        if hasattr(type(impl), name):
            return getattr(impl, name)
        impl._lazy_init()
        if hasattr(impl._C, name):
            return getattr(impl._C, name)
        raise AttributeError(name)

    mod.__getattr__ = __getattr__
    mod._impl = impl
    return mod


def _autoload():
    """Entry point of the `torch.backends` group (reference:
    torch_spyre/__init__.py:140-163).  Touches no device."""
    if getattr(_autoload, "_ran", False):
        return
    _autoload._ran = True

    import torch

    _patch_tensor_for_spyre()
    torch.utils.rename_privateuse1_backend(DEVICE_NAME)
    torch._register_device_module(DEVICE_NAME, make_spyre_module())
    torch.utils.generate_methods_for_privateuse1_backend(
        for_tensor=True, for_module=True, for_storage=True)

    from torch_spyre._inductor import _autoload as ts_autoload

    ts_autoload()


# Installed packages are registered by torch itself through the
# `torch.backends` entry point at `import torch`; importing the package (the
# in-tree case, with no entry point) registers it as well.
_autoload()
