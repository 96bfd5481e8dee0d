"""Tensor.__repr__ for spyre tensors.

Same behaviour as the reference (torch_spyre/_monkey_patch.py:16-48): the
tensor is printed through a copy to the CPU and the device string is
rewritten to the spyre device, so `str(t)` matches what CPU printing gives
plus `device='spyre:0'`.
"""


def _patch_tensor_for_spyre():
    import torch

    if getattr(torch.Tensor, "_spyre_repr_patched", False):
        return

    orig_repr = torch.Tensor.__repr__

    def spyre_aware_repr(self, *args, **kwargs):
        dev = getattr(self, "device", None)
        if dev is None or dev.type != "spyre":
            return orig_repr(self, *args, **kwargs)
        try:
            text = orig_repr(self.to("cpu"), *args, **kwargs)
        except Exception:  # printing must not raise for a live tensor
            return (f"SpyreTensor(shape={tuple(self.shape)}, dtype={self.dtype}, "
                    f"device={self.device})")
        dev_s = f"device='{self.device}'"
        if "device=" in text:
            return text.replace("device='cpu'", dev_s)
        if text.endswith(")"):
            return text[:-1] + f", {dev_s})"
        return text + f" ({dev_s})"

    torch.Tensor.__repr__ = spyre_aware_repr
    torch.Tensor._spyre_repr_patched = True
