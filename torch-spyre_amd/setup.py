"""Packaging of torch_spyre for MI355X.

The native pieces are built in-tree by build.py (hipcc for the gfx950 kernel
library, g++ for the PrivateUse1 extension); this file ships them with the
Python package and registers the same `torch.backends` entry point as the
reference (setup.py:189-191), so `import torch` loads the backend.
"""

from setuptools import find_packages, setup

setup(
    name="torch_spyre",
    version="0.1.0",
    description="torch-spyre's PrivateUse1 'spyre' device on AMD MI355X (gfx950)",
    packages=find_packages(include=["torch_spyre", "torch_spyre.*"]),
    package_data={"torch_spyre": ["_C*.so", "lib/*.so"]},
    python_requires=">=3.10",
    entry_points={"torch.backends": ["torch_spyre = torch_spyre:_autoload"]},
)
