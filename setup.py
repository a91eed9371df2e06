"""Package root of the MI355X build: installs `fused_decode` from
fused-decode_amd/fused_decode with its built HIP library and tile table
(run `python fused-decode_amd/build.py` first)."""

from setuptools import setup

setup(
    name="fused-decode-amd",
    version="0.2.0",
    description="fused-decode's decode operators as HIP kernels for MI355X (gfx950)",
    package_dir={"fused_decode": "fused-decode_amd/fused_decode"},
    packages=["fused_decode"],
    package_data={"fused_decode": ["*.so", "*.json"]},
    python_requires=">=3.10",
    install_requires=["torch", "numpy"],
)
