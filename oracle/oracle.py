"""ctypes bindings for the CPU oracle (liborc.so) and the reference build
(oracle/_ref/libxlref.so). TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liborc.so")
REFLIB = os.path.join(HERE, "_ref", "libxlref.so")

Q8K_BYTES = 292
Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
assert Q8K_DTYPE.itemsize == Q8K_BYTES

TYPES = {"IQ2_XXS": 16, "IQ2_XS": 17, "IQ1_M": 29}
BLOCK_BYTES = {16: 66, 17: 74, 29: 56}

_P = C.c_void_p
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load(path):
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run make -C {HERE}")
    return C.CDLL(path)


class Oracle:
    def __init__(self, path: str = LIB):
        L = self.lib = _load(path)
        L.orc_quantize_row.argtypes = [_f32p, C.c_int, _P]
        L.orc_dot.argtypes = [C.c_int, _u8p, _P, C.c_int]
        L.orc_dot.restype = C.c_float
        L.orc_block_partials.argtypes = [C.c_int, _u8p, _P, C.c_int, _i32p]
        L.orc_integer_lane.argtypes = [C.c_int, _u8p, _P, C.c_int, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]
        L.orc_matrix_ints.argtypes = [C.c_int, _u8p, C.c_int, C.c_int, _P, _i32p, C.c_int]
        L.orc_lane_avx2.restype = C.c_int
        L.orc_lane_dot.argtypes = [C.c_int, _u8p, _P, C.c_int]
        L.orc_lane_dot.restype = C.c_float
        L.orc_lane_layer.argtypes = [C.c_int, _i32p, _P, C.c_int, C.c_int, _f32p, _i32p, _f32p, _f32p, C.c_float,
                                     C.c_int, np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")]
        L.orc_brute_block.argtypes = [C.c_int, _u8p, _P]
        L.orc_brute_block.restype = C.c_int64
        L.orc_matvec.argtypes = [C.c_int, _u8p, C.c_int, C.c_int, _P, _f32p, C.c_int]
        L.orc_swiglu.argtypes = [C.c_float, C.c_float, C.c_float]
        L.orc_swiglu.restype = C.c_float
        L.orc_expert.argtypes = [_i32p, _u8p, _u8p, _u8p, C.c_int, C.c_int, _f32p, _f32p, _P, _P, _P, C.c_int, C.c_float]
        L.orc_down_from_hidden.argtypes = [C.c_int, _u8p, C.c_int, C.c_int, _f32p, _f32p, C.c_int]
        L.orc_combine.argtypes = [_i32p, _f32p, C.c_int, _f32p, C.c_int, _P, _f32p]
        L.orc_route.argtypes = [_f32p, C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_float, _i32p, _f32p]
        _i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
        L.orc_quant32.argtypes = [_f32p, C.c_int, _i8p, _f32p]
        L.orc_row32.argtypes = [C.c_int, _u8p, C.c_int, _i8p, _f32p]
        L.orc_row32.restype = C.c_float
        L.orc_matvec32.argtypes = [C.c_int, _u8p, C.c_int, C.c_int, _i8p, _f32p, _f32p]
        L.orc_row_bytes32.argtypes = [C.c_int, C.c_int]
        L.orc_row_bytes32.restype = C.c_int
        L.orc_dequant32.argtypes = [C.c_int, _u8p, C.c_int, np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")]
        L.orc_hc_post.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p]
        L.orc_hc_pre_norm.argtypes = [_f32p, _f32p, _P, C.c_int, C.c_int, C.c_int, C.c_float, _f32p]
        L.orc_expert32.argtypes = [_i32p, _u8p, _u8p, _u8p, C.c_int, C.c_int, _f32p, _f32p, _P, _P, _P, C.c_float]
        L.orc_gen_key.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_gen_key.restype = C.c_uint64
        L.orc_gen_block.argtypes = [C.c_int, C.c_uint64, C.c_uint64, _u8p]
        L.orc_gen_matrix.argtypes = [C.c_int, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, C.c_int, _u8p]
        L.orc_codebook.argtypes = [C.c_int, _u64p]
        L.orc_ksigns.argtypes = [C.c_int]
        L.orc_ksigns.restype = C.c_uint8
        L.orc_half.argtypes = [C.c_uint16]
        L.orc_half.restype = C.c_float
        L.orc_nearest.argtypes = [C.c_float]
        L.orc_nearest.restype = C.c_int

    # -- Q8_K ------------------------------------------------------------
    def quantize(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        assert x.size % 256 == 0
        out = np.zeros(x.size // 256, dtype=Q8K_DTYPE)
        self.lib.orc_quantize_row(x, x.size, out.ctypes.data)
        return out

    # -- dots ------------------------------------------------------------
    def dot(self, t: int, row: np.ndarray, act: np.ndarray) -> float:
        return float(self.lib.orc_dot(t, np.ascontiguousarray(row), act.ctypes.data, act.size))

    def block_partials(self, t: int, row: np.ndarray, act: np.ndarray) -> np.ndarray:
        out = np.zeros(act.size * (2 if t == 29 else 1), dtype=np.int32)
        self.lib.orc_block_partials(t, np.ascontiguousarray(row), act.ctypes.data, act.size, out)
        return out

    def matrix_ints(self, t: int, w: np.ndarray, n: int, k: int, act: np.ndarray, threads: int = 8) -> np.ndarray:
        """[n, k/256] block integers of an AoS matrix against Q8_K blocks act
        (IQ1_M: 8 * main + delta, the integer the device decoders form)."""
        act = np.ascontiguousarray(act)
        assert act.size == k // 256
        out = np.zeros((n, k // 256), np.int32)
        self.lib.orc_matrix_ints(t, np.ascontiguousarray(w).reshape(-1), n, k, act.ctypes.data, out.reshape(-1), threads)
        return out

    # -- the AVX2 CPU lane (cpu_lane.c) ----------------------------------
    def lane_avx2(self) -> bool:
        return bool(self.lib.orc_lane_avx2())

    def lane_dot(self, t: int, row: np.ndarray, act: np.ndarray) -> float:
        return float(self.lib.orc_lane_dot(t, np.ascontiguousarray(row), act.ctypes.data, act.size))

    def lane_layer(self, types, mats, ids, w, x, dim, ff, threads=1, limit=0.0, phases=None):
        """One routed layer on the AVX2 lane: types [k, 3], mats a list of k
        (gate, up, down) AoS arrays; phases (5 float64, added to): q1, gate_up,
        q2, down, combine ns."""
        k = len(ids)
        t = np.ascontiguousarray(types, dtype=np.int32).reshape(-1)
        flat = [np.ascontiguousarray(m) for tri in mats for m in tri]
        ptrs = (C.c_void_p * (3 * k))(*[m.ctypes.data for m in flat])
        out = np.zeros(dim, np.float32)
        ph = phases if phases is not None else np.zeros(5, np.float64)
        self.lib.orc_lane_layer(k, t, C.cast(ptrs, C.c_void_p), dim, ff, np.ascontiguousarray(x, dtype=np.float32),
                                np.ascontiguousarray(ids, dtype=np.int32), np.ascontiguousarray(w, dtype=np.float32),
                                out, float(limit), int(threads), ph)
        return out

    def integer_lane(self, t: int, block: np.ndarray, act_block: np.ndarray, lane: int):
        m, d = C.c_int32(), C.c_int32()
        self.lib.orc_integer_lane(t, np.ascontiguousarray(block), act_block.ctypes.data, lane, C.byref(m), C.byref(d))
        return m.value, d.value

    def brute_block(self, t: int, block: np.ndarray, act_block: np.ndarray) -> int:
        return int(self.lib.orc_brute_block(t, np.ascontiguousarray(block), act_block.ctypes.data))

    def matvec(self, t: int, w: np.ndarray, n: int, k: int, act: np.ndarray, threads: int = 8) -> np.ndarray:
        y = np.zeros(n, dtype=np.float32)
        self.lib.orc_matvec(t, np.ascontiguousarray(w).reshape(-1), n, k, act.ctypes.data, y, threads)
        return y

    def swiglu(self, g: float, u: float, limit: float = 0.0) -> float:
        return float(self.lib.orc_swiglu(g, u, limit))

    def expert(self, types, gate, up, down, dim, ff, x, threads=8, intermediates=False, limit=0.0):
        y = np.zeros(dim, dtype=np.float32)
        g = np.zeros(ff, dtype=np.float32); u = np.zeros(ff, dtype=np.float32); h = np.zeros(ff, dtype=np.float32)
        self.lib.orc_expert(np.asarray(types, dtype=np.int32), gate.reshape(-1), up.reshape(-1), down.reshape(-1),
                            dim, ff, np.ascontiguousarray(x, dtype=np.float32), y,
                            g.ctypes.data, u.ctypes.data, h.ctypes.data, threads, float(limit))
        return (y, g, u, h) if intermediates else y

    def down_from_hidden(self, t, down, dim, ff, h, threads=8):
        y = np.zeros(dim, dtype=np.float32)
        self.lib.orc_down_from_hidden(t, down.reshape(-1), dim, ff, np.ascontiguousarray(h, dtype=np.float32), y, threads)
        return y

    def combine(self, ids, w, rows, shared=None) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32); w = np.ascontiguousarray(w, dtype=np.float32)
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        k, dim = rows.shape
        out = np.zeros(dim, dtype=np.float32)
        sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
        self.lib.orc_combine(ids, w, k, rows.reshape(-1), dim, None if sh is None else sh.ctypes.data, out)
        return out

    # -- per32 arithmetic (the production HIP lane) ------------------------
    def quant32(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        q = np.zeros(x.size, np.int8); d = np.zeros(x.size // 32, np.float32)
        self.lib.orc_quant32(x, x.size, q, d)
        return q, d

    def row32(self, t, row, k, q, d) -> float:
        return float(self.lib.orc_row32(t, np.ascontiguousarray(row, dtype=np.uint8).reshape(-1), k,
                                        np.ascontiguousarray(q, dtype=np.int8), np.ascontiguousarray(d, dtype=np.float32)))

    def matvec32(self, t, w, n, k, q, d):
        y = np.zeros(n, np.float32)
        self.lib.orc_matvec32(t, np.ascontiguousarray(w, dtype=np.uint8).reshape(-1), n, k,
                              np.ascontiguousarray(q, dtype=np.int8), np.ascontiguousarray(d, dtype=np.float32), y)
        return y

    def row_bytes32(self, t, k) -> int:
        return int(self.lib.orc_row_bytes32(t, k))

    def dequant32(self, t, row, kb):
        out = np.zeros(32, np.float64)
        self.lib.orc_dequant32(t, np.ascontiguousarray(row, dtype=np.uint8).reshape(-1), kb, out)
        return out

    def hc_pre_norm(self, h, mix, w, eps=1e-6):
        """sycl/hc/core.hpp:74-80: h [T, H, D], mix [T, 8], w [D] or None -> x [T, D]."""
        T, H, D = (int(v) for v in np.shape(h))
        x = np.zeros((T, D), np.float32)
        wv = None if w is None else np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        self.lib.orc_hc_pre_norm(np.ascontiguousarray(h, dtype=np.float32).reshape(-1),
                                 np.ascontiguousarray(mix, dtype=np.float32).reshape(-1),
                                 None if wv is None else wv.ctypes.data, D, H, T, float(eps), x.reshape(-1))
        return x

    def hc_post(self, y, res, post, comb, D, H, T):
        """sycl/hc/core.hpp:81-86: y [T, D], res [T, H, D], post [T, 8], comb [T, 64] -> [T, H, D]."""
        out = np.zeros((T, H, D), np.float32)
        self.lib.orc_hc_post(*(np.ascontiguousarray(a, dtype=np.float32).reshape(-1) for a in (y, res, post, comb)),
                             D, H, T, out.reshape(-1))
        return out

    def expert32(self, types, gate, up, down, dim, ff, x, intermediates=False, limit=0.0):
        y = np.zeros(dim, np.float32)
        g = np.zeros(ff, np.float32); u = np.zeros(ff, np.float32); h = np.zeros(ff, np.float32)
        self.lib.orc_expert32(np.asarray(types, dtype=np.int32), gate.reshape(-1), up.reshape(-1), down.reshape(-1), dim,
                              ff, np.ascontiguousarray(x, dtype=np.float32), y, g.ctypes.data, u.ctypes.data,
                              h.ctypes.data, float(limit))
        return (y, g, u, h) if intermediates else y

    def route(self, logits, k, scale=1.0, bias=None):
        """route.cpp:15-37 for logits [T, n] (or [n]): ids, weights [T, k]."""
        lg = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
        T, n = lg.shape
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        ids = np.zeros((T, k), np.int32); w = np.zeros((T, k), np.float32)
        self.lib.orc_route(lg.reshape(-1), n, None if b is None else b.ctypes.data, n, T, k, scale, ids.reshape(-1),
                           w.reshape(-1))
        return ids, w

    # -- generator -------------------------------------------------------
    def gen_key(self, seed, layer, expert, role) -> int:
        return int(self.lib.orc_gen_key(seed, layer, expert, role))

    def gen_block(self, t, key, blk) -> np.ndarray:
        out = np.zeros(BLOCK_BYTES[t], dtype=np.uint8)
        self.lib.orc_gen_block(t, key, blk, out)
        return out

    def gen_matrix(self, t, seed, layer, expert, role, n, k) -> np.ndarray:
        out = np.zeros(n * (k // 256) * BLOCK_BYTES[t], dtype=np.uint8)
        self.lib.orc_gen_matrix(t, seed, layer, expert, role, n, k, out)
        return out

    def gen_expert(self, types, seed, layer, expert, dim, ff):
        """AoS bytes of (gate, up, down) of one expert; roles 0, 1, 2."""
        return (self.gen_matrix(types[0], seed, layer, expert, 0, ff, dim),
                self.gen_matrix(types[1], seed, layer, expert, 1, ff, dim),
                self.gen_matrix(types[2], seed, layer, expert, 2, dim, ff))

    def codebook(self, which: int) -> np.ndarray:
        out = np.zeros((256, 512, 2048)[which], dtype=np.uint64)
        self.lib.orc_codebook(which, out)
        return out

    def ksigns(self) -> np.ndarray:
        return np.array([self.lib.orc_ksigns(i) for i in range(128)], dtype=np.uint8)


class Reference:
    """The reference's own q8k_core.hpp / core.hpp / other_combine.hpp, compiled
    from /root/reference into oracle/_ref (absent where the reference is)."""

    def __init__(self, path: str = REFLIB):
        L = self.lib = _load(path)
        L.ref_quant_block.argtypes = [_f32p, _P]
        L.ref_dot.argtypes = [C.c_int, _u8p, _P, C.c_int]
        L.ref_dot.restype = C.c_float
        L.ref_integer_lane.argtypes = [C.c_int, _u8p, _P, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.ref_swiglu.argtypes = [C.c_float, C.c_float, C.c_float]
        L.ref_swiglu.restype = C.c_float
        L.ref_half.argtypes = [C.c_uint16]
        L.ref_half.restype = C.c_float
        L.ref_nearest.argtypes = [C.c_float]
        L.ref_nearest.restype = C.c_int
        L.ref_table.argtypes = [C.c_int, _u64p]
        L.ref_decode.argtypes = [C.c_int, _u8p, C.c_int, _i32p, _i32p, C.POINTER(C.c_float), _P]
        L.ref_hc_post.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p]
        L.ref_hc_pre_norm.argtypes = [_f32p, _f32p, _P, C.c_int, C.c_int, C.c_int, C.c_float, _f32p]
        L.ref_matvec.argtypes = [C.c_int, _u8p, C.c_int, C.c_int, _P, _f32p, C.c_int]
        L.ref_combine.argtypes = [_i32p, _f32p, C.c_int, _f32p, C.c_int, _f32p, _f32p]
        L.ref_route.argtypes = [_f32p, C.c_int, _f32p, C.c_int, C.c_int, C.c_int, C.c_float, _i32p, _f32p]
        L.ref_row32.argtypes = [C.c_int, _u8p, C.c_int, np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS"), _f32p]
        L.ref_row32.restype = C.c_float
        L.ref_expert.argtypes = [_i32p, _u8p, _u8p, _u8p, C.c_int, C.c_int, _f32p, _f32p, C.c_int, C.c_float]

    @staticmethod
    def available() -> bool:
        return os.path.exists(REFLIB)

    def quantize(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 256)
        out = np.zeros(x.shape[0], dtype=Q8K_DTYPE)
        for b in range(x.shape[0]):
            self.lib.ref_quant_block(np.ascontiguousarray(x[b]), out[b:b + 1].ctypes.data)
        return out

    def dot(self, t, row, act) -> float:
        return float(self.lib.ref_dot(t, np.ascontiguousarray(row), act.ctypes.data, act.size))

    def integer_lane(self, t, block, act_block, lane):
        m, d = C.c_int(), C.c_int()
        self.lib.ref_integer_lane(t, np.ascontiguousarray(block), act_block.ctypes.data, lane, C.byref(m), C.byref(d))
        return m.value, d.value

    def matvec(self, t, w, n, k, act, threads=8):
        y = np.zeros(n, dtype=np.float32)
        self.lib.ref_matvec(t, np.ascontiguousarray(w).reshape(-1), n, k, act.ctypes.data, y, threads)
        return y

    def swiglu(self, g, u, limit=0.0):
        return float(self.lib.ref_swiglu(g, u, limit))

    def table(self, which):
        out = np.zeros((256, 512, 2048, 128)[which], dtype=np.uint64)
        self.lib.ref_table(which, out)
        return out

    def decode(self, t, row, kb):
        q, s, d, _ = self.decode_full(t, row, kb)
        return q, s, d

    def decode_full(self, t, row, kb):
        """core.hpp decode: values, per-16 scales, d, per-16 min terms."""
        q = np.zeros(32, dtype=np.int32); s = np.zeros(2, dtype=np.int32); d = C.c_float()
        m = np.zeros(2, dtype=np.float32)
        self.lib.ref_decode(t, np.ascontiguousarray(row), kb, q, s, C.byref(d), m.ctypes.data)
        return q, s, d.value, m

    def hc_pre_norm(self, h, mix, w, eps=1e-6):
        T, H, D = (int(v) for v in np.shape(h))
        x = np.zeros((T, D), np.float32)
        wv = None if w is None else np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        self.lib.ref_hc_pre_norm(np.ascontiguousarray(h, dtype=np.float32).reshape(-1),
                                 np.ascontiguousarray(mix, dtype=np.float32).reshape(-1),
                                 None if wv is None else wv.ctypes.data, D, H, T, float(eps), x.reshape(-1))
        return x

    def hc_post(self, y, res, post, comb, D, H, T):
        out = np.zeros((T, H, D), np.float32)
        self.lib.ref_hc_post(*(np.ascontiguousarray(a, dtype=np.float32).reshape(-1) for a in (y, res, post, comb)),
                             D, H, T, out.reshape(-1))
        return out

    def expert(self, types, gate, up, down, dim, ff, x, threads=8, limit=0.0):
        y = np.zeros(dim, dtype=np.float32)
        self.lib.ref_expert(np.asarray(types, dtype=np.int32), gate.reshape(-1), up.reshape(-1), down.reshape(-1),
                            dim, ff, np.ascontiguousarray(x, dtype=np.float32), y, threads, float(limit))
        return y

    def route(self, logits, k, scale=1.0, bias=None):
        lg = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
        T, n = lg.shape
        b = np.zeros(n, np.float32) if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        ids = np.zeros((T, k), np.int32); w = np.zeros((T, k), np.float32)
        self.lib.ref_route(lg.reshape(-1), n, b, n, T, k, scale, ids.reshape(-1), w.reshape(-1))
        return ids, w

    def row32(self, t, row, k, q, d) -> float:
        return float(self.lib.ref_row32(t, np.ascontiguousarray(row, dtype=np.uint8).reshape(-1), k,
                                        np.ascontiguousarray(q, dtype=np.int8), np.ascontiguousarray(d, dtype=np.float32)))

    def combine(self, ids, w, rows, shared):
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        k, dim = rows.shape
        out = np.zeros(dim, dtype=np.float32)
        self.lib.ref_combine(np.ascontiguousarray(ids, dtype=np.int32), np.ascontiguousarray(w, dtype=np.float32), k,
                             rows.reshape(-1), dim, np.ascontiguousarray(shared, dtype=np.float32), out)
        return out
