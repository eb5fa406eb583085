"""Build the MI355X (gfx950) MXFP4 MLP extension in place.

    python setup.py build_ext --inplace

First compiles every ``tinyinfer_amd/csrc/*.hip`` with hipcc for gfx950 into
``tinyinfer_amd/libtinyinfer_mxfp4.so`` (the C ABI), then builds the torch
wrapper ``tinyinfer_amd._C`` from ``csrc/bind.cpp`` against it.  No CUDA
sources, no hipify step, no JIT cache.
"""

import os

from setuptools import setup
from torch.utils.cpp_extension import BuildExtension, CppExtension

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "tinyinfer_amd")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


class BuildHipThenTorch(BuildExtension):
    def run(self):
        import importlib.util

        spec = importlib.util.spec_from_file_location("_ti_build", os.path.join(PKG, "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        if not os.environ.get("TINYINFER_SKIP_HIP_LIB"):
            mod.build_hip_library()
        super().run()


setup(
    name="tinyinfer_amd",
    version="0.1.0",
    packages=["tinyinfer_amd"],
    ext_modules=[
        CppExtension(
            name="tinyinfer_amd._C",
            sources=["tinyinfer_amd/csrc/bind.cpp"],
            include_dirs=[os.path.join(ROOT, "include"), os.path.join(ROCM, "include")],
            define_macros=[("__HIP_PLATFORM_AMD__", "1")],
            library_dirs=[PKG, os.path.join(ROCM, "lib")],
            libraries=["tinyinfer_mxfp4", "amdhip64", "c10_hip"],
            extra_compile_args=["-O3", "-std=c++17"],
            extra_link_args=["-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"],
        )
    ],
    cmdclass={"build_ext": BuildHipThenTorch},
)
