"""Device op overrides used by Inductor's wrapper codegen for the spyre
device (reference: torch_spyre/utils/device_op_overrides.py:20-36, which has
no streams).  Generated wrappers synchronise and select devices through
torch.spyre; kernel runners launch on the spyre stream themselves."""

from __future__ import annotations

from torch._inductor.codegen.common import DeviceOpOverrides


class SpyreDeviceOpOverrides(DeviceOpOverrides):
    def import_get_raw_stream_as(self, name: str) -> str:
        return f"from torch_spyre._C import _stream_handle as {name}"

    def set_device(self, device_idx: int) -> str:
        return f"torch.spyre.set_device({device_idx})"

    def synchronize(self) -> str:
        return "torch.spyre.synchronize()"

    def device_guard(self, device_idx: int) -> str:
        return "contextlib.nullcontext()"
