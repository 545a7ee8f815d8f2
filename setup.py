"""Wheel build of the astra_cuda package (astra-cuda_amd/astra_cuda): compiles
libastra_market.so (the HIP engine, astra-cuda_amd/csrc) and the compiled binding
astra_cuda._C (csrc/bindings.cpp, against the installed torch) into the package
directory before the package files are collected.

    pip install --no-build-isolation .
"""
import importlib.util
import os

from setuptools import setup
from setuptools.command.build_py import build_py

HERE = os.path.dirname(os.path.abspath(__file__))


class BuildPyWithEngine(build_py):
    def run(self):
        path = os.path.join(HERE, "astra-cuda_amd", "astra_cuda", "build.py")
        spec = importlib.util.spec_from_file_location("astra_cuda_build", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)  # build.py imports only the standard library (and torch
        print("built", mod.build(verbose=True))  # for the binding)
        print("built", mod.build_binding(verbose=True))
        super().run()


setup(
    name="astra_cuda",
    version="0.0.2",
    description="MI355X-native (gfx950) VecMarket order-matching engine and high-low "
                "trading game, a drop-in for astra_cuda",
    python_requires=">=3.10",
    install_requires=["numpy", "torch"],
    package_dir={"": "astra-cuda_amd"},
    packages=["astra_cuda"],
    package_data={"astra_cuda": ["libastra_market.so", "_C*.so"]},
    cmdclass={"build_py": BuildPyWithEngine},
)
