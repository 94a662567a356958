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


class EntropyMLPEngine:
    """The fused MLP engine EE/test_engine.py:17-26 constructs and calls:

        eng = EntropyMLPEngine(gate_w, up_w, down_w, tau_low, tau_high)
        out = eng.forward(hidden, entropy)

    gate_w, up_w fp16 [Inter, H] and down_w fp16 [H, Inter] (nn.Linear
    layout).  The reference's extension never defines the class
    (EE/csrc/engine.cpp:202-216); its test times it against
    F.linear(F.silu(F.linear(x, gate_w)) * F.linear(x, up_w), down_w) under
    the dispatcher's tier choice (EE/test_engine.py:33-39).  Here the weights
    are quantised per output channel once (EE/python/dispatch.py:43-48) and
    each forward runs the tier's GEMMs, SiLU*up and the tier's re-quantisation
    of the intermediate in one C call (ee_mlp_forward), with gate and up as one
    [2*Inter, H] operand.

    entropy: a float picks one tier for the call by the dispatcher's strict
    compares (EE/python/dispatch.py:74-79; no host sync); a float32 tensor with
    one value per token routes each token to its own tier (no host sync).
    """

    def __init__(self, gate_w: torch.Tensor, up_w: torch.Tensor, down_w: torch.Tensor, tau_low: float = 2.0,
                 tau_high: float = 3.5):
        for name, w in (("gate_w", gate_w), ("up_w", up_w), ("down_w", down_w)):
            if not w.is_cuda:
                raise RuntimeError(f"{name} must be a GPU tensor")
            if w.dtype != torch.float16 or w.dim() != 2:
                raise RuntimeError(f"{name} must be a 2-D float16 tensor")
        F, H = gate_w.shape
        if tuple(up_w.shape) != (F, H) or tuple(down_w.shape) != (H, F):
            raise RuntimeError(f"shape mismatch: gate {tuple(gate_w.shape)}, up {tuple(up_w.shape)}, "
                               f"down {tuple(down_w.shape)}; expected [I, H], [I, H], [H, I]")
        if H % 16 or F % 32:
            raise RuntimeError("the hidden size must be a multiple of 16 and the intermediate size of 32 "
                               "(gate|up rows are interleaved in blocks of 32)")
        self.device = gate_w.device
        self.H, self.F = H, F
        self.tau_low, self.tau_high = float(tau_low), float(tau_high)
        dev = self.device
        g, u, d = (w.contiguous() for w in (gate_w, up_w, down_w))
        e = lambda shape, dt: torch.empty(shape, dtype=dt, device=dev)
        self.gu_i8, self.gu_f8, self.gu_f16, self.gu_scale = (e((2 * F, H), torch.int8), e((2 * F, H), torch.uint8),
                                                              e((2 * F, H), torch.float16), e(2 * F, torch.float32))
        self.dn_i8, self.dn_f8, self.dn_f16, self.dn_scale = (e((H, F), torch.int8), e((H, F), torch.uint8),
                                                              e((H, F), torch.float16), e(H, torch.float32))
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().ee_mlp_prepare(
                _lib.engine(), g.data_ptr(), u.data_ptr(), d.data_ptr(), H, F, H, H, F,
                self.gu_i8.data_ptr(), self.gu_f8.data_ptr(), self.gu_f16.data_ptr(), self.gu_scale.data_ptr(),
                self.dn_i8.data_ptr(), self.dn_f8.data_ptr(), self.dn_f16.data_ptr(), self.dn_scale.data_ptr(),
                _lib.stream_handle()))

    def tier(self, entropy: float):
        """The tier a scalar entropy selects (EE/python/dispatch.py:74-79)."""
        from .dispatch import tier_of
        return tier_of(float(entropy), self.tau_low, self.tau_high)

    def forward(self, hidden: torch.Tensor, entropy) -> torch.Tensor:
        if not hidden.is_cuda or hidden.device != self.device:
            raise RuntimeError(f"hidden must be on {self.device}")
        if hidden.dtype != torch.float16:
            raise RuntimeError("hidden must be float16")
        if hidden.shape[-1] != self.H:
            raise RuntimeError(f"hidden size mismatch: got {hidden.shape[-1]}, engine has {self.H}")
        x = hidden.reshape(-1, self.H)
        if x.stride(-1) != 1 or (x.shape[0] > 1 and x.stride(0) != self.H) or x.data_ptr() % 16:
            x = x.contiguous()
        M = x.shape[0]
        if M == 0:
            return torch.empty((*hidden.shape[:-1], self.H), dtype=torch.float16, device=self.device)
        h_rows = None
        if isinstance(entropy, torch.Tensor) and entropy.numel() > 1:
            if entropy.numel() != M:
                raise RuntimeError(f"per-token entropy needs {M} values, got {entropy.numel()}")
            h_rows = entropy.reshape(M).to(device=self.device, dtype=torch.float32).contiguous()
            e = 0.0
        else:
            e = float(entropy)
        out = torch.empty((M, self.H), dtype=torch.float16, device=self.device)
        L = _lib.lib()
        nbytes = L.ee_mlp_workspace_bytes(M, self.H, self.F, int(h_rows is not None))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)
        with torch.cuda.device(self.device):
            _lib.check(L.ee_mlp_forward(
                _lib.engine(), x.data_ptr(), self.H, M, self.H, self.F,
                self.gu_i8.data_ptr(), self.gu_f8.data_ptr(), self.gu_f16.data_ptr(), self.gu_scale.data_ptr(),
                self.dn_i8.data_ptr(), self.dn_f8.data_ptr(), self.dn_f16.data_ptr(), self.dn_scale.data_ptr(),
                e, h_rows.data_ptr() if h_rows is not None else None, self.tau_low, self.tau_high,
                out.data_ptr(), self.H, ws.data_ptr(), nbytes, _lib.stream_handle()))
        return out.reshape(*hidden.shape[:-1], self.H)

    __call__ = forward
