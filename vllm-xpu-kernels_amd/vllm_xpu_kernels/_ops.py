"""Loads the in-tree HIP library and its PyTorch op registration.

There is no fallback: if the built libraries are missing, importing this
module raises, so nothing can silently run a non-HIP path.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmi355moe.so")
TORCH_EXT_PATH = os.path.join(_HERE, "_mi355moe_torch.so")

if not (os.path.exists(LIB_PATH) and os.path.exists(TORCH_EXT_PATH)):
    raise ImportError(
        "vllm_xpu_kernels: the HIP libraries are not built "
        f"({LIB_PATH}, {TORCH_EXT_PATH}); run "
        "`python vllm-xpu-kernels_amd/build.py`")

torch.ops.load_library(TORCH_EXT_PATH)
lib = ctypes.CDLL(LIB_PATH)
lib.mi355moe_last_error.restype = ctypes.c_char_p
