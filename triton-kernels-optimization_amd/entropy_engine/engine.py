"""CubinEngine counterpart: one gfx950 GEMM code object launched through the C ABI.

Mirrors entropy_engine_cuda.CubinEngine (EE/csrc/engine.cpp:64-216; EE =
"entropy-engine (1)/entropy-engine" in the reference):
  CubinEngine(code_object_path, func_name, shared_mem, num_warps, block_m, block_n)
  CubinEngine.from_metadata(code_object_path, meta_json_path, func_name)
  engine.forward(a_int8, b_int8, a_scale, b_scale) -> fp16 [M, N]
Differences, all deliberate: the code object is a gfx950 ELF (*.hsaco)
loaded with hipModuleLoadData; num_warps counts wave64s; the launch goes on
torch's current stream (the reference used the NULL stream, engine.cpp:160);
the module is unloaded when the engine is garbage-collected (the reference
leaked it).  Reference kernel names (gemm_int8_kernel, ...) are accepted as
aliases of this build's symbols.  Errors raise RuntimeError with the
reference's messages ("a must be int8", "K mismatch: ...", "Missing key: X").
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib
from .kernels import prepare_weight

KERNEL_ALIASES = {
    "gemm_int8_kernel": "eek_gemm_i8",
}

DEFAULT_CODE_OBJECT = os.path.join(_lib.LIB_DIR, "gemm.hsaco")
DEFAULT_META = os.path.join(_lib.LIB_DIR, "gemm_int8_meta.json")


class CubinEngine:
    def __init__(self, cubin_path: str = DEFAULT_CODE_OBJECT, func_name: str = "gemm_int8_kernel",
                 shared_mem: int = 65536, num_warps: int = 4, block_m: int = 128, block_n: int = 128,
                 _handle: int | None = None):
        L = _lib.lib()
        self._handle = None
        if _handle is None:
            if not torch.cuda.is_available():
                raise RuntimeError("CubinEngine needs a ROCm GPU (gfx950); none is visible")
            torch.cuda.init()
            out = ctypes.c_void_p()
            _lib.check(L.ee_module_engine_create(os.fsencode(cubin_path), KERNEL_ALIASES.get(func_name, func_name).encode(),
                                                 shared_mem, num_warps, block_m, block_n, ctypes.byref(out)))
            _handle = out.value
        self._handle = _handle
        self.device = torch.device("cuda", torch.cuda.current_device())
        vals = [ctypes.c_int32() for _ in range(4)]
        _lib.check(L.ee_module_engine_info(self._handle, *[ctypes.byref(v) for v in vals]))
        self.shared_mem, self.num_warps, self.block_m, self.block_n = (v.value for v in vals)

    @classmethod
    def from_metadata(cls, cubin_path: str = DEFAULT_CODE_OBJECT, meta_json_path: str = DEFAULT_META,
                      func_name: str = "gemm_int8_kernel") -> "CubinEngine":
        if not torch.cuda.is_available():
            raise RuntimeError("CubinEngine needs a ROCm GPU (gfx950); none is visible")
        torch.cuda.init()
        out = ctypes.c_void_p()
        _lib.check(_lib.lib().ee_module_engine_from_metadata(
            os.fsencode(cubin_path), os.fsencode(meta_json_path),
            KERNEL_ALIASES.get(func_name, func_name).encode(), ctypes.byref(out)))
        return cls(_handle=out.value)

    def forward(self, a_int8: torch.Tensor, b_int8: torch.Tensor, a_scale: torch.Tensor,
                b_scale: torch.Tensor) -> torch.Tensor:
        """EE/csrc/engine.cpp:106-166: int8 A [M, K] (pre-quantised), int8 B
        [K, N], f32 scales [M], [N] -> fp16 C [M, N]."""
        if a_int8.dtype != torch.int8:
            raise RuntimeError("a must be int8")
        if b_int8.dtype != torch.int8:
            raise RuntimeError("b must be int8")
        if a_scale.dtype != torch.float32:
            raise RuntimeError("a_scale must be fp32")
        if b_scale.dtype != torch.float32:
            raise RuntimeError("b_scale must be fp32")
        if not a_int8.is_contiguous():
            raise RuntimeError("a must be contiguous")
        if not b_int8.is_contiguous():
            raise RuntimeError("b must be contiguous")
        M, K = a_int8.shape
        K2, N = b_int8.shape
        if K != K2:
            raise RuntimeError(f"K mismatch: a is [{M},{K}], b is [{K2},{N}]")
        if a_scale.numel() != M or b_scale.numel() != N:
            raise RuntimeError("scale length mismatch: a_scale must be [M], b_scale [N]")
        for t in (a_int8, b_int8, a_scale, b_scale):
            if t.device != self.device:
                raise RuntimeError(f"tensor on {t.device}, engine on {self.device}")
        b_nk = prepare_weight(b_int8, b_scale).i8
        out = torch.empty((M, N), dtype=torch.float16, device=self.device)
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().ee_module_engine_forward(
                self._handle, a_int8.data_ptr(), K, b_nk.data_ptr(), K, out.data_ptr(), N,
                a_scale.data_ptr(), b_scale.data_ptr(), M, N, K, _lib.stream_handle()))
        return out

    __call__ = forward

    def __del__(self):
        h, self._handle = getattr(self, "_handle", None), None
        if h is not None and _lib._lib is not None:
            try:
                _lib._lib.ee_module_engine_destroy(h)
            except Exception:
                pass


HsacoEngine = CubinEngine
