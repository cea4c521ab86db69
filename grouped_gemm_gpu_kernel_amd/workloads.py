"""Synthetic grouped-GEMM workloads.

Shapes, alpha and beta are drawn on the host with numpy's legacy RandomState
(its streams are frozen across numpy versions).  Matrix data is generated on
the GPU by the library's counter-hash fill kernels, so even the ~20 GB
long-tail set needs no host copy.  Every matrix is tightly packed (lda = k,
ldb = ldc = ldd = n, like the reference's generators,
bench/benchmark_grouped_gemm.cu:464-468) and starts on a 256-byte boundary of
one pool per operand; odd k or n therefore gives rows that start on 2-byte
boundaries, which the kernels handle.

Workloads (the benchmark configurations):
  plumbing16    16 problems, m, n, k uniform in [1, 256]; A, B, C uniform[-1, 1];
                alpha 1, beta 0.5
  mixed512      512 problems, m, n log-uniform in [64, 1024], k log-uniform in
                [64, 2048]; A, B, C uniform[-1, 1]; alpha uniform[0.5, 2], beta
                uniform[0, 1]
  dense64       64 problems 2048^3; A, B normal(0, 1/sqrt(2048)); C zero;
                alpha 1, beta 0
  moe64         64 groups, k 4096, n 14336, group sizes: 16384 tokens drawn
                from a Zipf(1.2) law over the experts (ranks permuted), then
                the 4 smallest groups are emptied into the largest so that some
                groups have m = 0; A, B normal(0, 0.02); no C; alpha 1, beta 0
  longtail4096  4096 problems in random order: 205 large (m, n uniform in
                [1024, 4096], k uniform in [1024, 8192]), the rest tiny (m, n, k
                uniform in [1, 64]); A, B, C uniform[-1, 1]; alpha 1, beta 1
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from .api import ProblemDesc

WORKLOADS = ("plumbing16", "mixed512", "dense64", "moe64", "longtail4096")
ALIGN = 256


@dataclass
class WorkloadSpec:
    name: str
    m: np.ndarray
    n: np.ndarray
    k: np.ndarray
    alpha: np.ndarray
    beta: np.ndarray
    ab_dist: tuple          # ("uniform", lo, hi) or ("normal", sigma)
    c_dist: Optional[tuple]  # ("uniform", lo, hi), ("zero",) or None (no C)
    seed: int
    config: str             # macro-tile the workload is quoted on

    @property
    def count(self) -> int:
        return int(self.m.size)

    def flops(self) -> float:
        return float(np.sum(2.0 * self.m.astype(np.float64) * self.n * self.k))

    def algorithmic_bytes(self) -> float:
        """A and B read once, C read when beta != 0, D written once, for m, n > 0."""
        m = self.m.astype(np.float64)
        n = self.n.astype(np.float64)
        k = self.k.astype(np.float64)
        live = (m > 0) & (n > 0)
        reads_c = (self.beta != 0) & (self.c_dist is not None) & (self.c_dist != ("zero",))
        per = 2 * m * k + 2 * k * n + 4 * m * n * (1 + reads_c.astype(np.float64))
        return float(np.sum(np.where(live, per, 0.0)))


def _log_uniform_int(rs: np.random.RandomState, lo: int, hi: int, size: int) -> np.ndarray:
    """floor(exp(u)), u uniform in [ln lo, ln(hi + 1)), clipped to [lo, hi]."""
    u = rs.uniform(math.log(lo), math.log(hi + 1), size)
    return np.clip(np.floor(np.exp(u)), lo, hi).astype(np.int32)


def make_spec(name: str, seed: int = 42) -> WorkloadSpec:
    rs = np.random.RandomState(seed)
    if name == "plumbing16":
        m = rs.randint(1, 257, 16).astype(np.int32)
        n = rs.randint(1, 257, 16).astype(np.int32)
        k = rs.randint(1, 257, 16).astype(np.int32)
        return WorkloadSpec(name, m, n, k, np.ones(16, np.float32), np.full(16, 0.5, np.float32),
                            ("uniform", -1.0, 1.0), ("uniform", -1.0, 1.0), seed, "128x64x32")
    if name == "mixed512":
        m = _log_uniform_int(rs, 64, 1024, 512)
        n = _log_uniform_int(rs, 64, 1024, 512)
        k = _log_uniform_int(rs, 64, 2048, 512)
        alpha = rs.uniform(0.5, 2.0, 512).astype(np.float32)
        beta = rs.uniform(0.0, 1.0, 512).astype(np.float32)
        return WorkloadSpec(name, m, n, k, alpha, beta, ("uniform", -1.0, 1.0), ("uniform", -1.0, 1.0),
                            seed, "128x64x32")
    if name == "dense64":
        full = np.full(64, 2048, np.int32)
        return WorkloadSpec(name, full.copy(), full.copy(), full.copy(), np.ones(64, np.float32),
                            np.zeros(64, np.float32), ("normal", 1.0 / math.sqrt(2048.0)), ("zero",), seed,
                            "128x64x32")
    if name == "moe64":
        experts, tokens = 64, 16384
        weights = np.arange(1, experts + 1, dtype=np.float64) ** -1.2
        weights /= weights.sum()
        probs = weights[rs.permutation(experts)]
        counts = rs.multinomial(tokens, probs).astype(np.int64)
        order = np.argsort(counts, kind="stable")
        largest = order[-1]
        for e in order[:4]:
            counts[largest] += counts[e]
            counts[e] = 0
        assert counts.sum() == tokens
        m = counts.astype(np.int32)
        return WorkloadSpec(name, m, np.full(experts, 14336, np.int32), np.full(experts, 4096, np.int32),
                            np.ones(experts, np.float32), np.zeros(experts, np.float32), ("normal", 0.02),
                            None, seed, "128x64x32")
    if name == "longtail4096":
        count, n_large = 4096, 205
        large = np.zeros(count, bool)
        large[rs.permutation(count)[:n_large]] = True
        m = rs.randint(1, 65, count)
        n = rs.randint(1, 65, count)
        k = rs.randint(1, 65, count)
        m[large] = rs.randint(1024, 4097, n_large)
        n[large] = rs.randint(1024, 4097, n_large)
        k[large] = rs.randint(1024, 8193, n_large)
        return WorkloadSpec(name, m.astype(np.int32), n.astype(np.int32), k.astype(np.int32),
                            np.ones(count, np.float32), np.ones(count, np.float32), ("uniform", -1.0, 1.0),
                            ("uniform", -1.0, 1.0), seed, "128x64x32")
    raise ValueError(f"unknown workload {name!r}; known: {WORKLOADS}")


def custom_spec(name: str, m, n, k, alpha=None, beta=None, ab_dist=("uniform", -1.0, 1.0),
                c_dist=("uniform", -1.0, 1.0), seed: int = 1, config: str = "128x64x32") -> WorkloadSpec:
    m = np.asarray(m, np.int32)
    n = np.asarray(n, np.int32)
    k = np.asarray(k, np.int32)
    cnt = m.size
    alpha = np.ones(cnt, np.float32) if alpha is None else np.asarray(alpha, np.float32)
    beta = np.zeros(cnt, np.float32) if beta is None else np.asarray(beta, np.float32)
    return WorkloadSpec(name, m, n, k, alpha, beta, ab_dist, c_dist, seed, config)


def _round_up(x: int, a: int = ALIGN) -> int:
    return (x + a - 1) // a * a


def _elems(rows: int, cols: int) -> int:
    return max(1, int(rows)) * max(1, int(cols)) if rows > 0 and cols > 0 else 1


class DeviceWorkload:
    """A workload's matrices on the current GPU: one torch pool per operand.

    Offsets are in elements of each pool; A/B pools are int16 holding binary16
    bits, C/D pools float32.  problems() gives the ProblemDesc list.
    """

    def __init__(self, spec: WorkloadSpec, device: str = "cuda"):
        import torch

        self.spec = spec
        cnt = spec.count
        self.a_off = np.zeros(cnt, np.int64)
        self.b_off = np.zeros(cnt, np.int64)
        self.c_off = np.zeros(cnt, np.int64)
        self.d_off = np.zeros(cnt, np.int64)
        a_tot = b_tot = c_tot = d_tot = 0
        for i in range(cnt):
            mi, ni, ki = int(spec.m[i]), int(spec.n[i]), int(spec.k[i])
            self.a_off[i] = a_tot
            a_tot += _round_up(_elems(mi, ki) * 2) // 2
            self.b_off[i] = b_tot
            b_tot += _round_up(_elems(ki, ni) * 2) // 2
            self.c_off[i] = c_tot
            c_tot += _round_up(_elems(mi, ni) * 4) // 4
            self.d_off[i] = d_tot
            d_tot += _round_up(_elems(mi, ni) * 4) // 4
        self.a = torch.empty(a_tot, dtype=torch.int16, device=device)
        self.b = torch.empty(b_tot, dtype=torch.int16, device=device)
        self.has_c = spec.c_dist is not None
        self.c = torch.empty(c_tot if self.has_c else 1, dtype=torch.float32, device=device)
        self.d = torch.empty(d_tot, dtype=torch.float32, device=device)
        stream = torch.cuda.current_stream().cuda_stream
        L = _lib.lib()
        for pool, sid in ((self.a, 1), (self.b, 2)):
            if spec.ab_dist[0] == "uniform":
                st = L.ggk_fill_uniform_f16(pool.data_ptr(), pool.numel(), spec.seed, sid, spec.ab_dist[1],
                                            spec.ab_dist[2], stream)
            else:
                st = L.ggk_fill_normal_f16(pool.data_ptr(), pool.numel(), spec.seed, sid, spec.ab_dist[1], stream)
            _lib.check(st, "fill A/B")
        if self.has_c:
            if spec.c_dist[0] == "uniform":
                st = L.ggk_fill_uniform_f32(self.c.data_ptr(), self.c.numel(), spec.seed, 3, spec.c_dist[1],
                                            spec.c_dist[2], stream)
            else:
                st = L.ggk_fill_f32(self.c.data_ptr(), self.c.numel(), 0.0, stream)
            _lib.check(st, "fill C")
        self.poison_d()
        torch.cuda.synchronize()

    def poison_d(self, value: float = float("nan")) -> None:
        import torch

        _lib.check(_lib.lib().ggk_fill_f32(self.d.data_ptr(), self.d.numel(), value,
                                           torch.cuda.current_stream().cuda_stream), "poison D")

    def problems(self) -> list:
        spec = self.spec
        a0, b0, c0, d0 = self.a.data_ptr(), self.b.data_ptr(), self.c.data_ptr(), self.d.data_ptr()
        out = []
        for i in range(spec.count):
            mi, ni, ki = int(spec.m[i]), int(spec.n[i]), int(spec.k[i])
            out.append(ProblemDesc(
                m=mi, n=ni, k=ki,
                a=a0 + int(self.a_off[i]) * 2, b=b0 + int(self.b_off[i]) * 2,
                c=(c0 + int(self.c_off[i]) * 4) if self.has_c else None,
                d=d0 + int(self.d_off[i]) * 4,
                lda=max(1, ki), ldb=max(1, ni), ldc=max(1, ni), ldd=max(1, ni),
                alpha=float(spec.alpha[i]), beta=float(spec.beta[i])))
        return out

    def tensors(self):
        """Per-problem torch views (a fp16 [m, k], b fp16 [k, n], c fp32 [m, n] or None, d fp32
        [m, n]) of the pools, for the torch binding."""
        import torch

        spec = self.spec
        a, b, c, d = [], [], [], []
        for i in range(spec.count):
            mi, ni, ki = int(spec.m[i]), int(spec.n[i]), int(spec.k[i])

            def view(pool, off, rows, cols, dtype):
                flat = pool[int(off):int(off) + rows * cols]
                return (flat.view(dtype) if dtype != pool.dtype else flat).view(rows, cols)

            a.append(view(self.a, self.a_off[i], mi, ki, torch.float16))
            b.append(view(self.b, self.b_off[i], ki, ni, torch.float16))
            c.append(view(self.c, self.c_off[i], mi, ni, torch.float32) if self.has_c else None)
            d.append(view(self.d, self.d_off[i], mi, ni, torch.float32))
        return a, b, c, d, [float(x) for x in spec.alpha], [float(x) for x in spec.beta]

    # Host copies of one problem's operands (tests and the CPU baseline).
    def host_a(self, i: int) -> np.ndarray:
        n = _elems(int(self.spec.m[i]), int(self.spec.k[i]))
        return self.a[int(self.a_off[i]):int(self.a_off[i]) + n].cpu().numpy().view(np.uint16)

    def host_b(self, i: int) -> np.ndarray:
        n = _elems(int(self.spec.k[i]), int(self.spec.n[i]))
        return self.b[int(self.b_off[i]):int(self.b_off[i]) + n].cpu().numpy().view(np.uint16)

    def host_c(self, i: int) -> Optional[np.ndarray]:
        if not self.has_c:
            return None
        n = _elems(int(self.spec.m[i]), int(self.spec.n[i]))
        return self.c[int(self.c_off[i]):int(self.c_off[i]) + n].cpu().numpy()

    def host_d(self, i: int) -> np.ndarray:
        n = _elems(int(self.spec.m[i]), int(self.spec.n[i]))
        return self.d[int(self.d_off[i]):int(self.d_off[i]) + n].cpu().numpy()

    def host_a_rows(self, i: int, rows: np.ndarray) -> np.ndarray:
        """Rows of A_i as uint16 [len(rows), k]."""
        k = int(self.spec.k[i])
        base = int(self.a_off[i])
        import torch

        idx = torch.as_tensor(base + rows.astype(np.int64)[:, None] * k + np.arange(k)[None, :],
                              device=self.a.device)
        return self.a[idx].cpu().numpy().view(np.uint16)

    def host_b_cols(self, i: int, cols: np.ndarray) -> np.ndarray:
        """Columns of B_i as uint16 [k, len(cols)]."""
        k, n = int(self.spec.k[i]), int(self.spec.n[i])
        base = int(self.b_off[i])
        import torch

        idx = torch.as_tensor(base + np.arange(k)[:, None] * n + cols.astype(np.int64)[None, :],
                              device=self.b.device)
        return self.b[idx].cpu().numpy().view(np.uint16)
