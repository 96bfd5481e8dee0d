"""torch.compile backend for the spyre device (MI355X).

Reference: torch_spyre/_inductor/__init__.py:23-98.  Registration is the
same (device interface, device op overrides, scheduling + wrapper codegen
for "spyre", the `torch.ops.spyre.*` custom ops with their decompositions
and lowerings, `Tensor.get_dci`); what the backend emits differs: fused HIP
kernels compiled by hiprtc for gfx950 (spyre_kernel.py), with matrix
products left to the eager MFMA kernels as extern calls.  Unlike the
reference no global Inductor setting is changed (its autoload rewrites
config, the AOT autograd entry, the choices handler and the pattern passes
for every device); the kernel-shape heuristics live in SpyreKernel and the
graph passes run through the per-device custom pass hook.
"""


class Unsupported(RuntimeError):
    def __init__(self, thing) -> None:
        super().__init__(f"Spyre backend does not support: {thing}")


DEVICE_NAME = "spyre"


def _autoload():
    from torch._dynamo.device_interface import register_interface_for_device
    from torch._inductor.codegen.common import (
        get_device_op_overrides,
        register_backend_for_device,
        register_device_op_overrides,
    )

    from torch_spyre.utils.device_interface import SpyreInterface
    from torch_spyre.utils.device_op_overrides import SpyreDeviceOpOverrides

    register_interface_for_device(DEVICE_NAME, SpyreInterface)
    # Inductor loads its built-in device op overrides lazily, only while its
    # table is empty; load them before adding "spyre" so compiling for the
    # CPU or other devices keeps working after this backend is registered.
    get_device_op_overrides("cpu")
    register_device_op_overrides(device=DEVICE_NAME, device_op_overrides=SpyreDeviceOpOverrides())

    from .scheduling import SpyreScheduling
    from .wrapper import SpyrePythonWrapperCodegen

    from .passes import CustomPostPasses
    from .stickify import install_spyre_tensors
    from . import customops  # noqa: F401  (registers torch.ops.spyre.*)
    from . import decompositions, lowering

    install_spyre_tensors()
    decompositions.register()
    lowering.register()
    register_backend_for_device(DEVICE_NAME, SpyreScheduling, SpyrePythonWrapperCodegen,
                                device_custom_pass=CustomPostPasses())
