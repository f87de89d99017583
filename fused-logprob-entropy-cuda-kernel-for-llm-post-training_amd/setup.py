"""Builds kernel_opt's compiled binding, kernel_opt/_lib/klp_torch*.so
(binding/klp_torch.cpp: a torch C++ extension over the C ABI of
kernel_opt/_lib/libkernel_opt_hip.so, which `make` builds first).

    python setup.py build_ext --inplace     # run by `make`

The extension finds libkernel_opt_hip.so next to itself (rpath $ORIGIN).
"""
import os

from setuptools import setup
from torch.utils.cpp_extension import BuildExtension, CppExtension

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "kernel_opt", "_lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

setup(
    name="kernel_opt_binding",
    ext_modules=[
        CppExtension(
            "kernel_opt._lib.klp_torch",
            [os.path.join("binding", "klp_torch.cpp")],
            include_dirs=[os.path.join(HERE, "..", "include"), os.path.join(ROCM, "include")],
            define_macros=[("__HIP_PLATFORM_AMD__", "1")],
            extra_compile_args=["-O2", "-g0", "-std=c++17", "-Wall"],
            library_dirs=[LIB_DIR, os.path.join(ROCM, "lib")],
            libraries=["kernel_opt_hip", "c10_hip", "amdhip64"],
            extra_link_args=["-Wl,-rpath,$ORIGIN", "-s"],
        )
    ],
    cmdclass={"build_ext": BuildExtension},
)
