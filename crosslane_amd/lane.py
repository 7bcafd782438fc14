"""ctypes binding of libcrosslane.so and the `Lane` class.

`Lane` keeps the reference lane's method names and meaning
(engine/strata/warm/runtime.hpp:10-16):

    warm_contains(layer, e)            -> bool
    warm_grouped()                     -> True (layer batches run in one call)
    warm_compute(layer, e, x)          -> y            (one expert)
    warm_compute_many(layer, ids, x)   -> [y_i ...]    (ids order)

plus `layer_forward`, which adds the caller's fixed-order combine
(warm_execute, engine/strata/warm/runtime.cpp:180-188), and device-resident
variants taking torch CUDA tensors. Errors raise `XLError`, as the reference
raises std::runtime_error from `require`.
"""
from __future__ import annotations

import ctypes as C
import os
import sys
from typing import Optional, Sequence

import numpy as np

IQ2_XXS, IQ2_XS, IQ1_M = 16, 17, 29
BLOCK_BYTES = {IQ2_XXS: 66, IQ2_XS: 74, IQ1_M: 56}
ABI_VERSION = 3
_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcrosslane.so")


class XLError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[xl {code}] {message}")
        self.code = code


class _Err(C.Structure):
    _fields_ = [("code", C.c_int32), ("message", C.c_char * 512)]


class _Config(C.Structure):
    _fields_ = [("struct_bytes", C.c_uint32), ("device", C.c_int32), ("dim", C.c_int32), ("ff", C.c_int32),
                ("n_layers", C.c_int32), ("n_experts", C.c_int32), ("max_picks", C.c_int32),
                ("max_tokens", C.c_int32), ("swiglu_limit", C.c_float)]


class _BankInfo(C.Structure):
    _fields_ = [("payload_bytes", C.c_uint64), ("allocated_bytes", C.c_uint64), ("workspace_bytes", C.c_uint64),
                ("n_layers", C.c_int32), ("n_experts", C.c_int32), ("generated", C.c_int32),
                ("reserved", C.c_int32)]


_P = C.c_void_p
_I32 = C.c_int32
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_ErrP = C.POINTER(_Err)

class _PackMeta(C.Structure):
    _fields_ = [("struct_bytes", C.c_uint32), ("dim", C.c_int32), ("ff", C.c_int32), ("n_layers", C.c_int32),
                ("n_experts", C.c_int32), ("top_k", C.c_int32), ("swiglu_limit", C.c_float)]


_SIGNATURES = {
    "xl_abi_version": (C.c_uint32, []),
    "xl_open": (_I32, [C.c_uint32, C.POINTER(_Config), C.POINTER(_P), _ErrP]),
    "xl_close": (None, [_P]),
    "xl_last_error": (_I32, [_P, _ErrP]),
    "xl_bank_create": (_I32, [_P, _i32p, _ErrP]),
    "xl_bank_generate": (_I32, [_P, C.c_uint64, _ErrP]),
    "xl_bank_upload": (_I32, [_P, _I32, _I32, _I32, _P, C.c_uint64, _ErrP]),
    "xl_bank_download": (_I32, [_P, _I32, _I32, _I32, _P, C.c_uint64, _ErrP]),
    "xl_bank_info_get": (_I32, [_P, C.POINTER(_BankInfo)]),
    "xl_contains": (_I32, [_P, _I32, _I32]),
    "xl_expert_forward": (_I32, [_P, _I32, _I32, _f32p, _f32p, _ErrP]),
    "xl_experts_forward": (_I32, [_P, _I32, _i32p, _I32, _f32p, _f32p, _ErrP]),
    "xl_layer_forward": (_I32, [_P, _I32, _i32p, _f32p, _I32, _f32p, _P, _f32p, _ErrP]),
    "xl_expert_trace": (_I32, [_P, _I32, _I32, _f32p, _P, _P, _P, _P, _P, _ErrP]),
    "xl_layer_forward_async": (_I32, [_P, _I32, _P, _P, _I32, _P, _P, _P, _P, _ErrP]),
    "xl_sync": (_I32, [_P, _P, _ErrP]),
    "xl_layer_trace_async": (_I32, [_P, _I32, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, C.POINTER(_I32), _P,
                                    _ErrP]),
    "xl_grouped_trace_async": (_I32, [_P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _ErrP]),
    "xl_combine_async": (_I32, [_P, _P, _P, _I32, _P, _I32, _P, _P, _P, _ErrP]),
    "xl_grouped_forward": (_I32, [_P, _I32, _I32, _I32, _i32p, _f32p, _f32p, _P, _f32p, _ErrP]),
    "xl_grouped_forward_async": (_I32, [_P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _ErrP]),
    "xl_route_async": (_I32, [_P, _P, _I32, _I32, _P, _I32, _I32, C.c_float, _P, _P, _P, _ErrP]),
    "xl_pack_meta_get": (_I32, [C.c_char_p, C.POINTER(_PackMeta), _ErrP]),
    "xl_pack_types": (_I32, [C.c_char_p, _I32, _I32, _I32, _i32p, _ErrP]),
    "xl_bank_load_pack": (_I32, [_P, C.c_char_p, _I32, _ErrP]),
    "xl_layer_forward_routed_async": (_I32, [_P, _I32, _P, _P, _I32, C.c_float, _P, _P, _P, _P, _ErrP]),
    "xl_grouped_forward_routed_async": (_I32, [_P, _I32, _I32, _P, _P, _I32, C.c_float, _P, _P, _P, _P, _ErrP]),
    "xl_quantize_q8k_async": (_I32, [_P, _P, _I32, _I32, _P, _P, _ErrP]),
    "xl_matvec_async": (_I32, [_P, _I32, _P, _I32, _I32, _P, _P, _P, _P, _ErrP]),
    "xl_swiglu_async": (_I32, [_P, _P, _P, _I32, C.c_float, _P, _P, _ErrP]),
    "xl_layer_forward_per32": (_I32, [_P, _I32, _i32p, _P, _I32, _f32p, _P, _P, _P, _ErrP]),
    "xl_layer_forward_per32_async": (_I32, [_P, _I32, _P, _P, _I32, _P, _P, _P, _P, _P, _ErrP]),
    "xl_quantize_per32_async": (_I32, [_P, _P, _I32, _I32, _P, _P, _P, _ErrP]),
    "xl_matvec_per32_async": (_I32, [_P, _I32, _P, _I32, _I32, _P, _P, _P, _P, _ErrP]),
    "xl_shared_work_bytes": (C.c_uint64, [_I32, _I32, _I32]),
    "xl_shared_forward_async": (_I32, [_P, _I32, _P, _I32, _P, _I32, _P, _I32, _I32, _P, _P, _P, C.c_uint64, _P,
                                       _ErrP]),
    "xl_shared_forward_noalloc": (_I32, [_P, _I32, _P, _I32, _P, _I32, _P, _I32, _I32, _P, _P, _P, _ErrP]),
    "xl_hc_post_async": (_I32, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _P, _P, _ErrP]),
    "xl_hc_pre_norm_async": (_I32, [_P, _P, _P, _P, _I32, _I32, _I32, C.c_float, _P, _P, _ErrP]),
    "xl_layer_forward_prenorm_async": (_I32, [_P, _I32, _P, _P, _I32, _P, _I32, _P, _P, C.c_float, _P, _P, _P, _P,
                                              _ErrP]),
    "xl_layer_forward_post_async": (_I32, [_P, _I32, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _ErrP]),
    "xl_moe_block_async": (_I32, [_P, _I32, _P, _P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, C.c_uint64,
                                  _P, _P, _P, _I32, _P, _P, _P, _ErrP]),
    "xl_profile_begin": (_I32, [_P, _I32, _ErrP]),
    "xl_profile_end": (_I32, [_P, _f32p, _I32, C.POINTER(_I32), C.POINTER(_I32), C.c_char_p, _I32, _ErrP]),
    "xl_profile_timeline": (_I32, [_P, _u64p, _I32, C.POINTER(_I32), _ErrP]),
    "xl_debug_set_launch_count": (_I32, [_P, C.c_uint32, _ErrP]),
    "xl_layer_forward_exact_async": (_I32, [_P, _I32, _P, _P, _I32, _P, _P, _P, _P, _ErrP]),
    "xl_debug_launch_counts": (_I32, [_P, np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS"), _I32, _ErrP]),
    "xl_planar_bytes": (C.c_uint64, [_I32, _I32, _I32]),
    "xl_repack": (_I32, [_I32, _I32, _I32, _P, _P]),
    "xl_restore": (_I32, [_I32, _I32, _I32, _P, _P]),
    "xl_generate_host": (_I32, [_I32, C.c_uint64, _I32, _I32, _I32, _I32, _I32, _P]),
    "xl_codebook": (_I32, [_I32, _u64p]),
}

_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """Loads libcrosslane.so from the package directory. No fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m crosslane_amd._build` "
                              "(or __graft_entry__.build()); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        if L.xl_abi_version() != ABI_VERSION:
            raise ImportError("libcrosslane.so ABI version differs from this binding")
        _lib = L
    return _lib


def _check(rc: int, err: _Err) -> None:
    if rc != 0:
        raise XLError(int(err.code or rc), err.message.decode(errors="replace"))


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    return int(t.data_ptr())


# ---- host utilities (no GPU) -------------------------------------------------
def planar_bytes(t: int, n: int, k: int) -> int:
    return int(lib().xl_planar_bytes(t, n, k))


def repack(t: int, n: int, k: int, aos: np.ndarray) -> np.ndarray:
    aos = np.ascontiguousarray(aos, dtype=np.uint8)
    assert aos.size == n * (k // 256) * BLOCK_BYTES[t]
    out = np.zeros(planar_bytes(t, n, k), dtype=np.uint8)
    rc = lib().xl_repack(t, n, k, aos.ctypes.data, out.ctypes.data)
    if rc:
        raise XLError(rc, "repack rejected its arguments")
    return out


def restore(t: int, n: int, k: int, planar: np.ndarray) -> np.ndarray:
    planar = np.ascontiguousarray(planar, dtype=np.uint8)
    out = np.zeros(n * (k // 256) * BLOCK_BYTES[t], dtype=np.uint8)
    rc = lib().xl_restore(t, n, k, planar.ctypes.data, out.ctypes.data)
    if rc:
        raise XLError(rc, "restore rejected its arguments")
    return out


def generate_host(t: int, seed: int, layer: int, expert: int, role: int, n: int, k: int) -> np.ndarray:
    out = np.zeros(n * (k // 256) * BLOCK_BYTES[t], dtype=np.uint8)
    rc = lib().xl_generate_host(t, seed, layer, expert, role, n, k, out.ctypes.data)
    if rc:
        raise XLError(rc, "generate_host rejected its arguments")
    return out


def codebook(which: int) -> np.ndarray:
    out = np.zeros((256, 512, 2048, 128)[which], dtype=np.uint64)
    rc = lib().xl_codebook(which, out)
    if rc:
        raise XLError(rc, "codebook index")
    return out


def pack_meta(pack_dir: str) -> dict:
    """Shape of a weight pack (ds4.txt): dim, ff, n_layers, n_experts, top_k, swiglu_limit."""
    m = _PackMeta(C.sizeof(_PackMeta))
    err = _Err()
    _check(lib().xl_pack_meta_get(os.fsencode(pack_dir), C.byref(m), C.byref(err)), err)
    return {f: getattr(m, f) for f, _ in _PackMeta._fields_[1:]}


def shared_work_bytes(dim: int, ff: int, T: int = 1) -> int:
    """Workspace bytes xl_shared_forward_async needs for T tokens."""
    return int(lib().xl_shared_work_bytes(dim, ff, T))


def pack_types(pack_dir: str, first_layer: int, n_layers: int, n_experts: int) -> np.ndarray:
    """Block types [n_layers, n_experts, 3] (gate, up, down) of a pack's layer window."""
    out = np.zeros((n_layers, n_experts, 3), np.int32)
    err = _Err()
    _check(lib().xl_pack_types(os.fsencode(pack_dir), first_layer, n_layers, n_experts, out.reshape(-1), C.byref(err)),
           err)
    return out


# ---- the lane ------------------------------------------------------------------
class Lane:
    """One context: a resident bank of n_layers x n_experts experts on one GPU.

    The *_async calls enqueue on `stream` (a raw HIP stream handle), by default
    on the context's own non-blocking stream. Tensors passed to them must stay
    alive until that stream has run the call (`sync(stream)`): PyTorch's caching
    allocator hands a freed tensor's memory to the next allocation on its own
    current stream at once, so a temporary such as `torch.tensor(...).cuda()`
    passed inline and followed by another allocation before the sync can be
    overwritten while the kernel reads it. Passing
    `stream=torch.cuda.current_stream().cuda_stream` orders the call with
    PyTorch's own work and allocations on that stream."""

    def __init__(self, dim: int, ff: int, n_layers: int, n_experts: int, types: np.ndarray,
                 max_picks: int = 8, max_tokens: int = 0, device: int = 0, swiglu_limit: float = 0.0):
        L = lib()
        cfg = _Config(C.sizeof(_Config), device, dim, ff, n_layers, n_experts, max_picks, max_tokens,
                      float(swiglu_limit))
        ctx = _P()
        err = _Err()
        _check(L.xl_open(ABI_VERSION, C.byref(cfg), C.byref(ctx), C.byref(err)), err)
        self._ctx = ctx
        self.dim, self.ff, self.n_layers, self.n_experts, self.max_picks = dim, ff, n_layers, n_experts, max_picks
        types = np.ascontiguousarray(types, dtype=np.int32).reshape(n_layers, n_experts, 3)
        self.types = types
        self._call("xl_bank_create", types.reshape(-1))

    # -- plumbing
    def _call(self, name: str, *args) -> None:
        err = _Err()
        _check(getattr(lib(), name)(self._ctx, *args, C.byref(err)), err)

    def close(self) -> None:
        if getattr(self, "_ctx", None):
            lib().xl_close(self._ctx)
            self._ctx = None

    def __del__(self):
        # At interpreter shutdown the HIP runtime (and torch's hold on it) may
        # already be torn down; process exit releases the device memory anyway,
        # so the context is left to it rather than closed into a dead runtime.
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- bank
    def generate(self, seed: int) -> None:
        self._call("xl_bank_generate", C.c_uint64(seed))

    def load_pack(self, pack_dir: str, first_layer: int = 0) -> None:
        """Uploads every expert of pack layers first_layer .. + n_layers - 1."""
        self._call("xl_bank_load_pack", os.fsencode(pack_dir), first_layer)

    def upload(self, layer: int, expert: int, role: int, aos: np.ndarray) -> None:
        aos = np.ascontiguousarray(aos, dtype=np.uint8)
        self._call("xl_bank_upload", layer, expert, role, aos.ctypes.data, C.c_uint64(aos.size))

    def download(self, layer: int, expert: int, role: int) -> np.ndarray:
        t = int(self.types[layer, expert, role])
        n, k = (self.ff, self.dim) if role < 2 else (self.dim, self.ff)
        out = np.zeros(n * (k // 256) * BLOCK_BYTES[t], dtype=np.uint8)
        self._call("xl_bank_download", layer, expert, role, out.ctypes.data, C.c_uint64(out.size))
        return out

    def info(self) -> dict:
        bi = _BankInfo()
        lib().xl_bank_info_get(self._ctx, C.byref(bi))
        return {f: getattr(bi, f) for f, _ in _BankInfo._fields_}

    # -- WarmRedirect surface
    def warm_contains(self, layer: int, e: int) -> bool:
        return bool(lib().xl_contains(self._ctx, layer, e))

    def warm_grouped(self) -> bool:
        return True

    def warm_compute(self, layer: int, e: int, x: np.ndarray) -> np.ndarray:
        y = np.zeros(self.dim, dtype=np.float32)
        self._call("xl_expert_forward", layer, e, np.ascontiguousarray(x, dtype=np.float32), y)
        return y

    def warm_compute_many(self, layer: int, ids: Sequence[int], x: np.ndarray) -> list:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        ys = np.zeros((ids.size, self.dim), dtype=np.float32)
        self._call("xl_experts_forward", layer, ids, ids.size, np.ascontiguousarray(x, dtype=np.float32),
                   ys.reshape(-1))
        return [ys[i] for i in range(ids.size)]

    def layer_forward(self, layer: int, ids: Sequence[int], weights: Sequence[float], x: np.ndarray,
                      shared: Optional[np.ndarray] = None) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        w = np.ascontiguousarray(weights, dtype=np.float32)
        out = np.zeros(self.dim, dtype=np.float32)
        sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
        self._call("xl_layer_forward", layer, ids, w, ids.size, np.ascontiguousarray(x, dtype=np.float32),
                   None if sh is None else sh.ctypes.data, out)
        return out

    def grouped_forward(self, layer: int, ids: np.ndarray, weights: np.ndarray, x: np.ndarray,
                        shared: Optional[np.ndarray] = None) -> np.ndarray:
        """T tokens at once: ids, weights [T, k]; x, shared [T, dim] -> out [T, dim]."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        T, k = ids.shape
        w = np.ascontiguousarray(weights, dtype=np.float32).reshape(T, k)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(T, self.dim)
        sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32).reshape(T, self.dim)
        out = np.zeros((T, self.dim), dtype=np.float32)
        self._call("xl_grouped_forward", layer, T, k, ids.reshape(-1), w.reshape(-1), x.reshape(-1),
                   None if sh is None else sh.ctypes.data, out.reshape(-1))
        return out

    def layer_forward_per32(self, layer: int, ids: Sequence[int], x: np.ndarray,
                            weights: Optional[Sequence[float]] = None, shared: Optional[np.ndarray] = None):
        """per32 layer (the reference's HIP lane arithmetic): returns (y [k, dim]
        per-pick down outputs, out [dim] their combine, or None without weights)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        y = np.zeros((ids.size, self.dim), dtype=np.float32)
        out = None if weights is None else np.zeros(self.dim, dtype=np.float32)
        w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
        sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
        self._call("xl_layer_forward_per32", layer, ids, None if w is None else w.ctypes.data, ids.size,
                   np.ascontiguousarray(x, dtype=np.float32), None if sh is None else sh.ctypes.data, y.ctypes.data,
                   None if out is None else out.ctypes.data)
        return y, out

    def expert_trace(self, layer: int, e: int, x: np.ndarray) -> dict:
        ff, dim = self.ff, self.dim
        g = np.zeros(ff, np.float32); u = np.zeros(ff, np.float32); h = np.zeros(ff, np.float32)
        q8h = np.zeros((ff // 256) * 292, np.uint8); y = np.zeros(dim, np.float32)
        self._call("xl_expert_trace", layer, e, np.ascontiguousarray(x, dtype=np.float32), g.ctypes.data,
                   u.ctypes.data, h.ctypes.data, q8h.ctypes.data, y.ctypes.data)
        return {"g": g, "u": u, "h": h, "q8h": q8h, "y": y}

    # -- device-resident (torch CUDA tensors)
    def layer_forward_async(self, layer: int, ids, w, x, out, shared=None, stream=None) -> None:
        self._call("xl_layer_forward_async", layer, _ptr(ids), _ptr(w), int(ids.numel()), _ptr(x), _ptr(shared),
                   _ptr(out), None if stream is None else int(stream))

    def layer_forward_exact_async(self, layer: int, ids, w, x, out, shared=None, stream=None) -> None:
        """xl_layer_forward_async with every float in the reference CPU lane's
        order (q8k_core.hpp:76-95): the reference's output bit for bit."""
        self._call("xl_layer_forward_exact_async", layer, _ptr(ids), _ptr(w), int(ids.numel()), _ptr(x), _ptr(shared),
                   _ptr(out), None if stream is None else int(stream))

    def layer_forward_prenorm_async(self, layer: int, ids, w, h, mix, norm_w, x, out, eps: float = 1e-6, shared=None,
                                    stream=None) -> None:
        """The layer on x = hc_pre_norm(h, mix, norm_w) of one token: h [H, dim]
        (or [1, H, dim]), mix [8], norm_w [dim] or None; x [dim] receives the
        normalized input (one launch when H == 1 and the layer has a streaming
        instance: the norm runs in its prologue)."""
        H = int(h.shape[-2]) if h.dim() >= 2 else 1
        self._call("xl_layer_forward_prenorm_async", layer, _ptr(ids), _ptr(w), int(ids.numel()), _ptr(h), H,
                   _ptr(mix), _ptr(norm_w), float(eps), _ptr(x), _ptr(shared), _ptr(out),
                   None if stream is None else int(stream))

    def layer_forward_post_async(self, layer: int, ids, w, x, out, res, post, comb, post_out, shared=None,
                                 stream=None) -> None:
        """The layer (out [dim], with shared added last) and hc_post of its output
        for one token: res and post_out [H, dim] (or [1, H, dim]; post_out may be
        res), post [8], comb [64]. One launch when the layer has a streaming
        instance: each workgroup applies hc_post to the rows it combines."""
        H = int(res.shape[-2]) if res.dim() >= 2 else 1
        self._call("xl_layer_forward_post_async", layer, _ptr(ids), _ptr(w), int(ids.numel()), _ptr(x), _ptr(shared),
                   _ptr(out), _ptr(res), _ptr(post), _ptr(comb), H, _ptr(post_out),
                   None if stream is None else int(stream))

    def moe_block_async(self, layer: int, ids, w, x, types, gate, up, down, ff: int, work, res, post, comb, out,
                        post_out, stream=None) -> None:
        """The MoE block of one token: the routed layer, the shared-expert FFN
        (types, gate, up, down, ff as shared_forward_async) added last, and
        hc_post of the sum: out [dim], res and post_out [H, dim] (post_out may be
        res), post [8], comb [64]; work >= shared_work_bytes(dim, ff, 1). The same
        bits as shared_forward_async then layer_forward_post_async with that row."""
        H = int(res.shape[-2]) if res.dim() >= 2 else 1
        self._call("xl_moe_block_async", layer, _ptr(ids), _ptr(w), int(ids.numel()), _ptr(x), int(types[0]),
                   _ptr(gate), int(types[1]), _ptr(up), int(types[2]), _ptr(down), ff, _ptr(work),
                   int(work.numel() * work.element_size()), _ptr(res), _ptr(post), _ptr(comb), H, _ptr(out),
                   _ptr(post_out), None if stream is None else int(stream))

    def layer_trace_async(self, layer: int, ids, w, x, out, q8x=None, q8h=None, h=None, ints=None, shared=None,
                          stream=None, y=None) -> int:
        """The single-launch layer call with its own Q8_K(x) / Q8_K(h) blocks (uint8
        tensors of 292-byte blocks), h, block integers and per-pick rows (y, k x dim,
        as its combine read them) written out; returns the kernel that ran (1
        streaming, 3 all-types)."""
        kern = _I32()
        self._call("xl_layer_trace_async", layer, _ptr(ids), _ptr(w), int(ids.numel()), _ptr(x), _ptr(shared),
                   _ptr(out), _ptr(q8x), _ptr(q8h), _ptr(h), _ptr(ints), _ptr(y), C.byref(kern),
                   None if stream is None else int(stream))
        return kern.value

    def grouped_trace_async(self, layer: int, ids, w, x, out, q8x=None, q8h=None, h=None, ints=None, shared=None,
                            stream=None, y=None) -> None:
        T, k = int(ids.shape[0]), int(ids.shape[1])
        self._call("xl_grouped_trace_async", layer, T, k, _ptr(ids), _ptr(w), _ptr(x), _ptr(shared), _ptr(out),
                   _ptr(q8x), _ptr(q8h), _ptr(h), _ptr(ints), _ptr(y), None if stream is None else int(stream))

    def combine_async(self, ids, w, rows, out, shared=None, stream=None) -> None:
        """xl_combine_async: out = fixed-order combine of rows [k, dim] (device tensors)."""
        k, dim = int(rows.shape[0]), int(rows.shape[1])
        self._call("xl_combine_async", _ptr(ids), _ptr(w), k, _ptr(rows), dim, _ptr(shared), _ptr(out),
                   None if stream is None else int(stream))

    def grouped_forward_async(self, layer: int, ids, w, x, out, shared=None, stream=None) -> None:
        """ids, w: [T, k] device tensors; x, out (and shared): [T, dim]."""
        T, k = int(ids.shape[0]), int(ids.shape[1])
        self._call("xl_grouped_forward_async", layer, T, k, _ptr(ids), _ptr(w), _ptr(x), _ptr(shared), _ptr(out),
                   None if stream is None else int(stream))

    def route_async(self, logits, k: int, ids, w, scale: float = 1.0, bias=None, stream=None) -> None:
        """logits: [T, n] device tensor; ids (int32), w: [T, k] device tensors."""
        T, n = int(logits.shape[0]), int(logits.shape[1])
        self._call("xl_route_async", _ptr(logits), T, int(logits.stride(0)), _ptr(bias), n, k, float(scale), _ptr(ids),
                   _ptr(w), None if stream is None else int(stream))

    def layer_forward_routed_async(self, layer: int, logits, k: int, x, out, scale: float = 1.0, bias=None,
                                   shared=None, stream=None) -> None:
        self._call("xl_layer_forward_routed_async", layer, _ptr(logits), _ptr(bias), k, float(scale), _ptr(x),
                   _ptr(shared), _ptr(out), None if stream is None else int(stream))

    def grouped_forward_routed_async(self, layer: int, logits, k: int, x, out, scale: float = 1.0, bias=None,
                                     shared=None, stream=None) -> None:
        self._call("xl_grouped_forward_routed_async", layer, int(logits.shape[0]), _ptr(logits), _ptr(bias), k,
                   float(scale), _ptr(x), _ptr(shared), _ptr(out), None if stream is None else int(stream))

    def sync(self, stream=None) -> None:
        self._call("xl_sync", None if stream is None else int(stream))

    def profile_begin(self, max_calls: int) -> None:
        self._call("xl_profile_begin", max_calls)

    def profile_end(self) -> dict:
        """Per-stage total milliseconds over the profiled calls: {name: ms}, calls."""
        ms = np.zeros(8, np.float32)
        ns, nc = _I32(), _I32()
        names = C.create_string_buffer(256)
        self._call("xl_profile_end", ms, 8, C.byref(ns), C.byref(nc), names, 256)
        keys = names.value.decode().split(",") if ns.value else []
        return {"calls": nc.value, "stages": {k: float(ms[i]) for i, k in enumerate(keys)}}

    def profile_timeline(self) -> np.ndarray:
        """Per-wave phase stamps (100 MHz) of the last profiled single-launch call: [waves, 32]."""
        out = np.zeros(1 << 16, np.uint64)
        n = _I32()
        self._call("xl_profile_timeline", out, out.size, C.byref(n))
        return out[: n.value].reshape(-1, 32)

    def debug_set_launch_count(self, launches: int) -> None:
        """Sets the single-launch kernels' launch counters (epoch / parity) as if
        `launches` launches had run: for testing their wrap at 2^32."""
        self._call("xl_debug_set_launch_count", C.c_uint32(launches & 0xFFFFFFFF))

    LAUNCH_KINDS = ("stream", "alltypes", "separate", "routed", "prenorm", "exact", "post", "block")   # XL_LAUNCH_* order

    def launch_counts(self) -> dict:
        """Layer calls so far by how they ran ({kind: count}, XL_LAUNCH_* kinds):
        which launch served a call (e.g. a routed call routed inside its launch)."""
        out = np.zeros(len(self.LAUNCH_KINDS), np.int64)
        self._call("xl_debug_launch_counts", out, out.size)
        return dict(zip(self.LAUNCH_KINDS, (int(v) for v in out)))

    def quantize_q8k_async(self, x, rows: int, k: int, q8k_out, stream=None) -> None:
        self._call("xl_quantize_q8k_async", _ptr(x), rows, k, _ptr(q8k_out), None if stream is None else int(stream))

    def layer_forward_per32_async(self, layer: int, ids, x, y, w=None, out=None, shared=None, stream=None) -> None:
        self._call("xl_layer_forward_per32_async", layer, _ptr(ids), _ptr(w), int(ids.numel()), _ptr(x), _ptr(shared),
                   _ptr(y), _ptr(out), None if stream is None else int(stream))

    def quantize_per32_async(self, x, rows: int, k: int, q, d, stream=None) -> None:
        self._call("xl_quantize_per32_async", _ptr(x), rows, k, _ptr(q), _ptr(d), None if stream is None else int(stream))

    def matvec_per32_async(self, t: int, planar, n: int, k: int, q, d, y, stream=None) -> None:
        self._call("xl_matvec_per32_async", t, _ptr(planar), n, k, _ptr(q), _ptr(d), _ptr(y),
                   None if stream is None else int(stream))

    def shared_forward_async(self, types, gate, up, down, ff: int, x, out, work, stream=None) -> None:
        """Shared-expert FFN of T tokens: x, out [T, dim] device tensors; gate, up,
        down raw ggml (dense) or planar (IQ) device bytes; work >= shared_work_bytes."""
        T = int(x.numel()) // self.dim
        self._call("xl_shared_forward_async", int(types[0]), _ptr(gate), int(types[1]), _ptr(up), int(types[2]),
                   _ptr(down), ff, T, _ptr(x), _ptr(out), _ptr(work), int(work.numel() * work.element_size()),
                   None if stream is None else int(stream))

    def shared_forward_noalloc(self, types, gate, up, down, ff: int, x, out, stream=None) -> None:
        """The shared-expert FFN with its intermediates in the library's static
        device scratch (no workspace, no allocation): x, out [T, dim]."""
        T = int(x.numel()) // self.dim
        self._call("xl_shared_forward_noalloc", int(types[0]), _ptr(gate), int(types[1]), _ptr(up), int(types[2]),
                   _ptr(down), ff, T, _ptr(x), _ptr(out), None if stream is None else int(stream))

    def hc_pre_norm_async(self, h, mix, w, x, eps: float = 1e-6, stream=None) -> None:
        """h [T, H, D], mix [T, 8], w [D] or None, x [T, D] device tensors."""
        T, H, D = (int(v) for v in h.shape)
        self._call("xl_hc_pre_norm_async", _ptr(h), _ptr(mix), _ptr(w), D, H, T, float(eps), _ptr(x),
                   None if stream is None else int(stream))

    def hc_post_async(self, y, res, post, comb, out, stream=None) -> None:
        """y [T, D], res / out [T, H, D], post [T, 8], comb [T, 64] device tensors."""
        T, H, D = (int(v) for v in res.shape)
        self._call("xl_hc_post_async", _ptr(y), _ptr(res), _ptr(post), _ptr(comb), D, H, T, _ptr(out),
                   None if stream is None else int(stream))

    def swiglu_async(self, g, u, h, limit: float = 0.0, stream=None) -> None:
        self._call("xl_swiglu_async", _ptr(g), _ptr(u), int(g.numel()), float(limit), _ptr(h),
                   None if stream is None else int(stream))

    def matvec_async(self, t: int, planar, n: int, k: int, x, y, partials=None, stream=None) -> None:
        self._call("xl_matvec_async", t, _ptr(planar), n, k, _ptr(x), _ptr(y), _ptr(partials),
                   None if stream is None else int(stream))
