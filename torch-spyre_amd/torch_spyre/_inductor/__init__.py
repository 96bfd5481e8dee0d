"""torch.compile backend for the spyre device (MI355X).

Reference: torch_spyre/_inductor/__init__.py:23-98.  Registration is the
same (device interface, device op overrides, scheduling + wrapper codegen
for "spyre"); what the backend emits differs: fused HIP kernels compiled by
hiprtc for gfx950 (spyre_kernel.py), with matrix products left to the eager
MFMA kernels as extern calls.  Unlike the reference no global Inductor
setting is changed (its autoload rewrites config, decompositions, the AOT
autograd entry and the pattern passes for every device).
"""


class Unsupported(RuntimeError):
    def __init__(self, thing) -> None:
        super().__init__(f"Spyre backend does not support: {thing}")


DEVICE_NAME = "spyre"


def _autoload():
    from torch._dynamo.device_interface import register_interface_for_device
    from torch._inductor.codegen.common import (
        register_backend_for_device,
        register_device_op_overrides,
    )

    from torch_spyre.utils.device_interface import SpyreInterface
    from torch_spyre.utils.device_op_overrides import SpyreDeviceOpOverrides

    register_interface_for_device(DEVICE_NAME, SpyreInterface)
    register_device_op_overrides(device=DEVICE_NAME, device_op_overrides=SpyreDeviceOpOverrides())

    from .scheduling import SpyreScheduling
    from .wrapper import SpyrePythonWrapperCodegen

    register_backend_for_device(DEVICE_NAME, SpyreScheduling, SpyrePythonWrapperCodegen)
