"""Device name of the backend (reference: torch_spyre/constants.py:15)."""

DEVICE_NAME = "spyre"
