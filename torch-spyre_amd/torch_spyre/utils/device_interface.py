"""Dynamo device interface of the spyre device (reference:
SpyreInterface, torch_spyre/utils/device_interface.py:25-53, which reports
fake properties "dd2" / 32 processors).  Here the properties are the real
ones of the MI355X read through torch_spyre._C."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch
from torch._dynamo.device_interface import DeviceInterface


@dataclass(frozen=True)
class SpyreDeviceProperties:
    type: str
    index: int
    name: str
    gcnArchName: str
    multi_processor_count: int
    total_memory: int
    warp_size: int


def _idx(device) -> int:
    if device is None:
        return -1
    if isinstance(device, torch.device):
        return -1 if device.index is None else device.index
    if isinstance(device, str):
        device = torch.device(device)
        return -1 if device.index is None else device.index
    return int(device)


class SpyreInterface(DeviceInterface):
    class Worker:
        @staticmethod
        def set_device(device: int):
            torch.spyre.set_device(device)

        @staticmethod
        def current_device() -> int:
            return torch.spyre.current_device()

        @staticmethod
        def get_device_properties(device=None):
            from torch_spyre import _C

            p = _C.get_device_properties(_idx(device))
            idx = _idx(device)
            return SpyreDeviceProperties(
                type="spyre", index=0 if idx < 0 else idx, name=p["name"],
                gcnArchName=p["gcnArchName"], multi_processor_count=p["multi_processor_count"],
                total_memory=p["total_memory"], warp_size=p["warp_size"])

    @staticmethod
    def is_available() -> bool:
        return torch.spyre.is_available()

    @staticmethod
    def device_count() -> int:
        return torch.spyre.device_count()

    @staticmethod
    def current_device() -> int:
        return torch.spyre.current_device()

    @staticmethod
    def set_device(device) -> None:
        torch.spyre.set_device(_idx(device) if _idx(device) >= 0 else 0)

    @staticmethod
    def synchronize(device=None) -> None:
        torch.spyre.synchronize()

    @staticmethod
    def get_raw_stream(device_idx: int) -> int:
        from torch_spyre import _C

        return _C._stream_handle(device_idx)

    @classmethod
    def get_device_properties(cls, device=None):
        return cls.Worker.get_device_properties(device)

    @staticmethod
    def get_compute_capability(device=None) -> Any:
        return "gfx950"

    @staticmethod
    def is_bf16_supported(including_emulation: bool = False) -> bool:
        return True

    @staticmethod
    def memory_allocated(device=None) -> int:
        return torch.spyre.memory_allocated()
