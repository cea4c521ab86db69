"""ctypes binding of the CPU oracle (oracle/liboracle.so, built by `make -C oracle`).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, as the expected answer or the timed CPU baseline.  The
product package never imports it.  Function semantics and reference citations
are in oracle/gg_oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_i = ctypes.c_int
_ip = ctypes.POINTER(ctypes.c_int)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_fp = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)


class MT19937(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint32 * 624), ("index", ctypes.c_int)]


_SIGS = {
    "go_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "go_f32_to_f16_rne": (ctypes.c_uint16, [ctypes.c_float]),
    "go_f32_to_f16_array": (None, [_fp, _u16p, ctypes.c_int64]),
    "go_f16_to_f32_array": (None, [_u16p, _fp, ctypes.c_int64]),
    "go_mt_seed": (None, [ctypes.POINTER(MT19937), ctypes.c_uint32]),
    "go_mt_next": (ctypes.c_uint32, [ctypes.POINTER(MT19937)]),
    "go_uniform_int": (_i, [ctypes.POINTER(MT19937), _i, _i]),
    "go_uniform_real_f32": (ctypes.c_float, [ctypes.POINTER(MT19937), ctypes.c_float, ctypes.c_float]),
    "go_bench_shapes": (_i, [ctypes.c_char_p, _i, ctypes.c_uint32, _ip, _ip, _ip]),
    "go_bench_shapes_lists": (None, [_i, ctypes.c_uint32, _ip, _i, _ip, _i, _ip, _i, _ip, _ip, _ip]),
    "go_reference_test_inputs": (None, [_i, _ip, _ip, _ip, ctypes.c_uint32, _fp, _fp, _i64p, _i64p, _i64p,
                                        _u16p, _u16p, _fp]),
    "go_tile_count": (_i, [_i, _i, _i, _i]),
    "go_prepare": (_i, [_i, _ip, _ip, _ip, _i, _i, _i, _ip, _ip]),
    "go_find_problem": (_i, [_ip, _i, _i]),
    "go_map_tiles": (None, [_i, _ip, _ip, _ip]),
    "go_grid_ctas": (_i, [_i, _i, _i, _i]),
    "go_gemm": (None, [_i, _i, _i, _u16p, _i, _u16p, _i, _fp, _i, ctypes.c_float, ctypes.c_float, _fp, _i]),
    "go_gemm_omp": (None, [_i, _i, _i, _u16p, _i, _u16p, _i, _fp, _i, ctypes.c_float, ctypes.c_float, _fp, _i,
                           _i]),
    "go_gemm_element": (ctypes.c_float, [_i, _i, _i, _u16p, _i, _u16p, _i, _fp, _i, ctypes.c_float,
                                         ctypes.c_float]),
    "go_gemm_samples": (None, [_i, _ip, _u16p, _i64p, _u16p, _i64p, _fp, _fp, _fp, _fp]),
    "go_total_flops": (ctypes.c_double, [_i, _ip, _ip, _ip]),
    "go_tail_work_share": (ctypes.c_double, [_i, _ip, _ip, _i]),
    "go_omp_max_threads": (_i, []),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", os.fspath(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _ints(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().go_f16_to_f32_array(_p(h, _u16p), _p(out, _fp), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().go_f32_to_f16_array(_p(f, _fp), _p(out, _u16p), f.size)
    return out


class Mt19937:
    def __init__(self, seed: int = 5489):
        self._s = MT19937()
        lib().go_mt_seed(ctypes.byref(self._s), seed)

    def next(self) -> int:
        return lib().go_mt_next(ctypes.byref(self._s))

    def uniform_int(self, lo: int, hi: int) -> int:
        return lib().go_uniform_int(ctypes.byref(self._s), lo, hi)

    def uniform_real(self, lo: float, hi: float) -> float:
        return lib().go_uniform_real_f32(ctypes.byref(self._s), lo, hi)


def bench_shapes(workload: str, count: int, seed: int):
    m = np.zeros(count, np.int32)
    n = np.zeros(count, np.int32)
    k = np.zeros(count, np.int32)
    if lib().go_bench_shapes(workload.encode(), count, seed, _p(m, _ip), _p(n, _ip), _p(k, _ip)) != 0:
        raise ValueError(workload)
    return m, n, k


def bench_shapes_lists(count: int, seed: int, m_values, n_values, k_values):
    """The small/mixed recipe over given candidate lists (gg_oracle.h)."""
    lists = [np.ascontiguousarray(v, np.int32) for v in (m_values, n_values, k_values)]
    m, n, k = (np.zeros(count, np.int32) for _ in range(3))
    lib().go_bench_shapes_lists(count, seed, _p(lists[0], _ip), lists[0].size, _p(lists[1], _ip), lists[1].size,
                                _p(lists[2], _ip), lists[2].size, _p(m, _ip), _p(n, _ip), _p(k, _ip))
    return m, n, k


def reference_test_inputs(m, n, k, seed: int = 20260328):
    """Per problem: (alpha, beta, A uint16, B uint16, C float32) exactly as the reference test
    draws them (tests/test_correctness.cu:106-150)."""
    m, n, k = _ints(m), _ints(n), _ints(k)
    cnt = m.size
    al, bl, cl = (np.zeros(cnt, np.int64) for _ in range(3))
    alpha = np.zeros(cnt, np.float32)
    beta = np.zeros(cnt, np.float32)
    L = lib()
    L.go_reference_test_inputs(cnt, _p(m, _ip), _p(n, _ip), _p(k, _ip), seed, _p(alpha, _fp), _p(beta, _fp),
                               _p(al, _i64p), _p(bl, _i64p), _p(cl, _i64p), None, None, None)
    a = np.zeros(int(al.sum()), np.uint16)
    b = np.zeros(int(bl.sum()), np.uint16)
    c = np.zeros(int(cl.sum()), np.float32)
    L.go_reference_test_inputs(cnt, _p(m, _ip), _p(n, _ip), _p(k, _ip), seed, _p(alpha, _fp), _p(beta, _fp),
                               _p(al, _i64p), _p(bl, _i64p), _p(cl, _i64p), _p(a, _u16p), _p(b, _u16p),
                               _p(c, _fp))
    out, ao, bo, co = [], 0, 0, 0
    for i in range(cnt):
        out.append((float(alpha[i]), float(beta[i]), a[ao:ao + al[i]], b[bo:bo + bl[i]], c[co:co + cl[i]]))
        ao += int(al[i])
        bo += int(bl[i])
        co += int(cl[i])
    return out


def tile_count(m: int, n: int, cta_m: int, cta_n: int) -> int:
    return lib().go_tile_count(m, n, cta_m, cta_n)


def prepare(m, n, k, cta_m: int, cta_n: int, mode: int):
    """(sorted_to_original, tile_offsets, total_tiles)."""
    m, n, k = _ints(m), _ints(n), _ints(k)
    cnt = m.size
    perm = np.zeros(max(1, cnt), np.int32)
    offs = np.zeros(cnt + 1, np.int32)
    total = lib().go_prepare(cnt, _p(m, _ip), _p(n, _ip), _p(k, _ip), cta_m, cta_n, mode, _p(perm, _ip),
                             _p(offs, _ip))
    return perm[:cnt], offs, total


def find_problem(offsets, tile: int) -> int:
    offs = _ints(offsets)
    return lib().go_find_problem(_p(offs, _ip), offs.size - 1, tile)


def map_tiles(sorted_tiles_n, offsets) -> np.ndarray:
    tn = _ints(sorted_tiles_n)
    offs = _ints(offsets)
    total = int(offs[-1])
    out = np.zeros(3 * max(1, total), np.int32)
    lib().go_map_tiles(tn.size, _p(tn, _ip), _p(offs, _ip), _p(out, _ip))
    return out[:3 * total].reshape(total, 3)


def grid_ctas(total_tiles: int, persistent_ctas: int, sm_count: int, active_blocks: int) -> int:
    return lib().go_grid_ctas(total_tiles, persistent_ctas, sm_count, active_blocks)


def gemm(m: int, n: int, k: int, a: np.ndarray, lda: int, b: np.ndarray, ldb: int, c: Optional[np.ndarray],
         ldc: int, alpha: float, beta: float, ldd: Optional[int] = None, threads: Optional[int] = None):
    """D (float32, m x ldd) of the reference host GEMM; threads=None runs the literal
    single-thread loop, otherwise the OpenMP i-k-j form (bit-identical)."""
    ldd = n if ldd is None else ldd
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    d = np.zeros(max(1, m * ldd), np.float32)
    cp = None
    if c is not None:
        c = np.ascontiguousarray(c, dtype=np.float32)
        cp = _p(c, _fp)
    if threads is None:
        lib().go_gemm(m, n, k, _p(a, _u16p), lda, _p(b, _u16p), ldb, cp, ldc, alpha, beta, _p(d, _fp), ldd)
    else:
        lib().go_gemm_omp(m, n, k, _p(a, _u16p), lda, _p(b, _u16p), ldb, cp, ldc, alpha, beta, _p(d, _fp), ldd,
                          threads)
    return d


def gemm_element(i: int, j: int, k: int, a: np.ndarray, lda: int, b: np.ndarray, ldb: int,
                 c: Optional[np.ndarray], ldc: int, alpha: float, beta: float) -> float:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    cp = None
    if c is not None:
        c = np.ascontiguousarray(c, dtype=np.float32)
        cp = _p(c, _fp)
    return lib().go_gemm_element(i, j, k, _p(a, _u16p), lda, _p(b, _u16p), ldb, cp, ldc, alpha, beta)


def gemm_samples(k, a: np.ndarray, a_start, b: np.ndarray, b_start, c, alpha, beta) -> np.ndarray:
    """Elements of the reference host GEMM given as (row of A, column of B) pairs: sample s is
    alpha[s] * sum_kk A[kk] B[kk] + beta[s] * c[s] over k[s] values at a[a_start[s]:] and
    b[b_start[s]:] (go_gemm_samples)."""
    k = _ints(k)
    cnt = k.size
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    a_start = np.ascontiguousarray(a_start, dtype=np.int64)
    b_start = np.ascontiguousarray(b_start, dtype=np.int64)
    assert a_start.size == cnt and b_start.size == cnt
    assert cnt == 0 or (int((a_start + k).max()) <= a.size and int((b_start + k).max()) <= b.size)
    alpha = np.ascontiguousarray(alpha, dtype=np.float32)
    beta = np.ascontiguousarray(beta, dtype=np.float32)
    cp = None
    if c is not None:
        c = np.ascontiguousarray(c, dtype=np.float32)
        cp = _p(c, _fp)
    out = np.zeros(max(1, cnt), np.float32)
    lib().go_gemm_samples(cnt, _p(k, _ip), _p(a, _u16p), _p(a_start, _i64p), _p(b, _u16p), _p(b_start, _i64p), cp,
                          _p(alpha, _fp), _p(beta, _fp), _p(out, _fp))
    return out[:cnt]


def total_flops(m, n, k) -> float:
    m, n, k = _ints(m), _ints(n), _ints(k)
    return lib().go_total_flops(m.size, _p(m, _ip), _p(n, _ip), _p(k, _ip))


def tail_work_share(sorted_k, offsets, cta_k: int) -> float:
    sk = _ints(sorted_k)
    offs = _ints(offsets)
    return lib().go_tail_work_share(sk.size, _p(sk, _ip), _p(offs, _ip), cta_k)


def omp_max_threads() -> int:
    return lib().go_omp_max_threads()
