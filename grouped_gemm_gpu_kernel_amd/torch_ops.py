"""PyTorch binding: the grouped GEMM on lists of torch tensors.

    d_i = alpha_i * a_i @ b_i + beta_i * c_i      for every i, in one persistent launch

a_i: float16 [m_i, k_i], b_i: float16 [k_i, n_i], c_i: float32 [m_i, n_i] or None, d_i: float32
[m_i, n_i]; products accumulate in float32 (the contract of the reference's ProblemDesc,
include/grouped_gemm/grouped_gemm.cuh:18-35).  Rows may be padded (a row stride above the row
length, e.g. a column slice of a wider tensor); elements inside a row must be contiguous.

Two forms:
* run_grouped_gemm(a, b, c, alpha, beta, ...) -- one call, the reference's run_grouped_gemm_once
  (src/grouped_gemm.cu:1279-1291): prepares, uploads, launches on the current stream and waits for
  it, because the executor's device buffers are released before it returns.  Registered as the
  custom op torch.ops.grouped_gemm_amd.grouped_gemm.
* GroupedGemmPlan(a, b, c, d, ...) -- prepare and upload once, then run() any number of times on
  any stream without host synchronisation, as the reference's GroupedGemmExecutor is used
  (include/grouped_gemm/grouped_gemm.cuh:94-115).  The plan holds its tensors; refill them in place
  between runs.

All work runs in the HIP library (lib/libgrouped_gemm_amd.so); there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Union

import numpy as np
import torch

from . import _lib
from .api import GroupedGemmExecutor, KernelConfig, ProblemDesc, SortMode, prepare_problem_set

Scalars = Union[float, Sequence[float]]

_OP_NAME = "grouped_gemm_amd::grouped_gemm"
_placeholders: dict = {}


def _placeholder(device: torch.device) -> int:
    """A valid device address for operands with no elements (the library rejects null a/b/d
    pointers even where nothing is read, src/grouped_gemm.cu:1304-1307)."""
    key = (device.type, device.index)
    if key not in _placeholders:
        _placeholders[key] = torch.zeros(64, dtype=torch.float32, device=device)
    return _placeholders[key].data_ptr()


def _row_stride(t: torch.Tensor) -> int:
    rows, cols = t.shape
    if rows <= 1 or t.numel() == 0:  # the stride of an empty or one-row matrix is never used
        return max(1, cols)
    return t.stride(0)


def _check_matrix(t: torch.Tensor, name: str, dtype: torch.dtype, shape, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    rows, cols = t.shape
    if t.numel() == 0:
        return
    if cols > 1 and t.stride(1) != 1:
        raise ValueError(f"{name} must have contiguous rows (stride(1) == 1)")
    if rows > 1 and t.stride(0) < max(1, cols):
        raise ValueError(f"{name} rows overlap (stride(0) < shape[1])")


def _per_problem(values: Scalars, count: int, name: str) -> list:
    if isinstance(values, (int, float)):
        return [float(values)] * count
    values = [float(v) for v in values]
    if len(values) != count:
        raise ValueError(f"{name} has {len(values)} entries for {count} problems")
    return values


def _problems(a, b, c, d, alpha, beta):
    count = len(a)
    if len(b) != count or len(d) != count or (c is not None and len(c) != count):
        raise ValueError("a, b, c and d must hold one tensor per problem")
    if count == 0:
        return []
    device = a[0].device
    if device.type != "cuda":
        raise ValueError(f"tensors must be on a GPU, got {device}")
    alpha = _per_problem(alpha, count, "alpha")
    beta = _per_problem(beta, count, "beta")
    dummy = _placeholder(device)
    problems = []
    for i in range(count):
        _check_matrix(a[i], f"a[{i}]", torch.float16, None, device)
        m, k = a[i].shape
        _check_matrix(b[i], f"b[{i}]", torch.float16, None, device)
        if b[i].shape[0] != k:
            raise ValueError(f"b[{i}] has {b[i].shape[0]} rows, a[{i}] has {k} columns")
        n = b[i].shape[1]
        _check_matrix(d[i], f"d[{i}]", torch.float32, (m, n), device)
        ci = None if c is None else c[i]
        if ci is not None:
            _check_matrix(ci, f"c[{i}]", torch.float32, (m, n), device)
        problems.append(ProblemDesc(
            m=m, n=n, k=k,
            a=a[i].data_ptr() or dummy, b=b[i].data_ptr() or dummy,
            c=(ci.data_ptr() or dummy) if ci is not None else None,
            d=d[i].data_ptr() or dummy,
            lda=_row_stride(a[i]), ldb=_row_stride(b[i]),
            ldc=_row_stride(ci) if ci is not None else max(1, n), ldd=_row_stride(d[i]),
            alpha=alpha[i], beta=beta[i]))
    return problems


# gg_problem_desc (include/grouped_gemm_amd.h) as a numpy record: one array of them is passed to the
# C ABI as is.
_DESC_DTYPE = np.dtype([("m", "<i4"), ("n", "<i4"), ("k", "<i4"), ("_pad", "<i4"), ("a", "<u8"), ("b", "<u8"),
                        ("c", "<u8"), ("d", "<u8"), ("lda", "<i4"), ("ldb", "<i4"), ("ldc", "<i4"),
                        ("ldd", "<i4"), ("alpha", "<f4"), ("beta", "<f4")])
assert _DESC_DTYPE.itemsize == ctypes.sizeof(_lib.GGProblemDesc)


def _ld(shape, stride) -> int:
    """_row_stride from a shape and stride already read."""
    rows, cols = shape
    if rows <= 1 or rows * cols == 0:
        return max(1, cols)
    return stride[0]


def _problem_table(a, b, c, d, alpha, beta) -> np.ndarray:
    """The problems of tensor lists as gg_problem_desc records, with the checks of _problems: each
    tensor's metadata is read once, in bulk, and any failed check is reported by _problems' own
    per-tensor messages."""
    count = len(a)
    if len(b) != count or len(d) != count or (c is not None and len(c) != count):
        raise ValueError("a, b, c and d must hold one tensor per problem")
    table = np.zeros(count, _DESC_DTYPE)
    if count == 0:
        return table
    device = a[0].device
    if device.type != "cuda":
        raise ValueError(f"tensors must be on a GPU, got {device}")
    cs = list(c) if c is not None else [None] * count
    f16, f32 = torch.float16, torch.float32
    try:
        sa = [t.shape for t in a]
        sb = [t.shape for t in b]
        sd = [t.shape for t in d]
        ok = (all(t.dtype is f16 and t.device == device for t in a) and
              all(t.dtype is f16 and t.device == device for t in b) and
              all(t.dtype is f32 and t.device == device for t in d) and
              all(t is None or (t.dtype is f32 and t.device == device) for t in cs) and
              all(len(x) == 2 and len(y) == 2 and x[1] == y[0] for x, y in zip(sa, sb)) and
              all(z == (x[0], y[1]) for x, y, z in zip(sa, sb, sd)) and
              all(t is None or t.shape == z for t, z in zip(cs, sd)))
        if ok:
            ta = [t.stride() for t in a]
            tb = [t.stride() for t in b]
            td = [t.stride() for t in d]
            tc = [t.stride() if t is not None else None for t in cs]
            # rows contiguous and not overlapping (see _check_matrix)
            for shapes, strides in ((sa, ta), (sb, tb), (sd, td)):
                ok = ok and all((x[1] <= 1 or s[1] == 1 or x[0] * x[1] == 0) and
                                (x[0] <= 1 or s[0] >= max(1, x[1]) or x[0] * x[1] == 0)
                                for x, s in zip(shapes, strides))
            ok = ok and all(t is None or ((z[1] <= 1 or s[1] == 1 or z[0] * z[1] == 0) and
                                          (z[0] <= 1 or s[0] >= max(1, z[1]) or z[0] * z[1] == 0))
                            for t, s, z in zip(cs, tc, sd))
    except (AttributeError, TypeError):
        ok = False
    if not ok:
        _problems(a, b, c, d, alpha, beta)  # raises with the failed check's message
        raise ValueError("tensor lists do not describe grouped GEMM problems")
    dummy = _placeholder(device)
    table["m"] = [x[0] for x in sa]
    table["k"] = [x[1] for x in sa]
    table["n"] = [x[1] for x in sb]
    table["a"] = [t.data_ptr() or dummy for t in a]
    table["b"] = [t.data_ptr() or dummy for t in b]
    table["d"] = [t.data_ptr() or dummy for t in d]
    table["c"] = [(t.data_ptr() or dummy) if t is not None else 0 for t in cs]
    table["lda"] = [_ld(x, s) for x, s in zip(sa, ta)]
    table["ldb"] = [_ld(x, s) for x, s in zip(sb, tb)]
    table["ldd"] = [_ld(x, s) for x, s in zip(sd, td)]
    table["ldc"] = [_ld(z, s) if t is not None else max(1, z[1]) for t, s, z in zip(cs, tc, sd)]
    table["alpha"] = _per_problem(alpha, count, "alpha")
    table["beta"] = _per_problem(beta, count, "beta")
    return table


class GroupedGemmPlan:
    """A prepared grouped GEMM over fixed tensors: prepare_problem_set + executor build once,
    run() per use.  Runs are stream-ordered and must not overlap each other (one scheduler state
    per plan, as one per executor in the reference)."""

    def __init__(self, a: Sequence[torch.Tensor], b: Sequence[torch.Tensor],
                 c: Optional[Sequence[Optional[torch.Tensor]]], d: Sequence[torch.Tensor],
                 alpha: Scalars = 1.0, beta: Scalars = 0.0, *, sort_mode: int = SortMode.kByK,
                 config: Optional[KernelConfig] = None):
        self.config = config if config is not None else KernelConfig.named("128x64x32")
        self.problems = _problems(a, b, c, d, alpha, beta)
        self._tensors = (list(a), list(b), None if c is None else list(c), list(d))
        self.prepared = prepare_problem_set(self.problems, self.config, sort_mode)
        self.executor = GroupedGemmExecutor()
        self.device = a[0].device if len(a) else None
        if self.problems:
            with torch.cuda.device(self.device):
                _lib.check(self.executor.build(self.prepared, self.config), "GroupedGemmExecutor.build")

    @property
    def outputs(self) -> list:
        return self._tensors[3]

    def run(self, stream: Optional[torch.cuda.Stream] = None) -> list:
        if not self.problems:
            return self.outputs
        with torch.cuda.device(self.device):
            stream = stream if stream is not None else torch.cuda.current_stream(self.device)
            _lib.check(self.executor.run(stream), "GroupedGemmExecutor.run")
        return self.outputs

    def close(self) -> None:
        self.executor.close()


def run_grouped_gemm(a: Sequence[torch.Tensor], b: Sequence[torch.Tensor],
                     c: Optional[Sequence[Optional[torch.Tensor]]] = None, alpha: Scalars = 1.0,
                     beta: Scalars = 0.0, *, sort_mode: int = SortMode.kByK,
                     config: Optional[KernelConfig] = None,
                     out: Optional[Sequence[torch.Tensor]] = None) -> list:
    """One grouped launch on the current stream; returns d (allocated unless given as out).
    Waits for the launch before returning (see the module docstring)."""
    if out is None:
        if len(a) and len(b) != len(a):
            raise ValueError("a and b must hold one tensor per problem")
        out = [torch.empty((ai.shape[0], bi.shape[1] if bi.dim() == 2 else 0), dtype=torch.float32,
                           device=ai.device) for ai, bi in zip(a, b)]
    # One C call (prepare, build, launch, wait, release) on a table read from the tensors in bulk.
    table = _problem_table(a, b, c, out, alpha, beta)
    if len(table) == 0:
        return list(out)
    config = config if config is not None else KernelConfig.named("128x64x32")
    device = a[0].device
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        status = _lib.lib().gg_run_grouped_gemm_once(
            table.ctypes.data_as(ctypes.POINTER(_lib.GGProblemDesc)), len(table), int(sort_mode),
            ctypes.byref(config.to_c()), stream or None)
    _lib.check(status, "run_grouped_gemm_once")
    return list(out)


# ---------------------------------------------------------------- mixture of experts

class MoeGroupedGemmPlan:
    """The grouped GEMM of a mixture-of-experts layer with device-side token counts:

        d[rows of e] = alpha * a[rows of e] @ b[e] + beta * c[rows of e]     for every expert e

    a: float16 [T, K], the tokens grouped by expert (expert e owns rows [r_e, r_e + counts[e]),
    r_e = sum of the counts before e); b: float16 [E, K, N]; d (and c): float32 [T, N].  The
    problem set is prepared on the GPU from the int32 counts tensor at every run() (see
    ggk_moe_prepare): no host synchronisation, no allocation, so runs can be captured in a CUDA/HIP
    graph and replayed with new counts.  Rows past T are never touched: counts that add up to more
    are clamped (status() reports it)."""

    def __init__(self, a: torch.Tensor, b: torch.Tensor, d: torch.Tensor, c: Optional[torch.Tensor] = None,
                 alpha: float = 1.0, beta: float = 0.0, *, sort_mode: int = SortMode.kByTiles,
                 config: Optional[KernelConfig] = None):
        from .api import MoeGroupedGemm, MoeLayout

        if a.device.type != "cuda":
            raise ValueError(f"tensors must be on a GPU, got {a.device}")
        if b.dim() != 3:
            raise ValueError(f"b must be [experts, K, N], got shape {tuple(b.shape)}")
        experts, k, n = b.shape
        _check_matrix(a, "a", torch.float16, None, a.device)
        if a.shape[1] != k:
            raise ValueError(f"a has {a.shape[1]} columns, b has K = {k}")
        rows = a.shape[0]
        _check_matrix(d, "d", torch.float32, (rows, n), a.device)
        if c is not None:
            _check_matrix(c, "c", torch.float32, (rows, n), a.device)
        if b.dtype != torch.float16 or b.device != a.device:
            raise TypeError("b must be float16 on the same device as a")
        if n > 1 and b.stride(2) != 1:
            raise ValueError("b[e] must have contiguous rows")
        if b.numel() and experts > 1 and b.stride(0) < 1:
            raise ValueError("b experts overlap")
        self.device = a.device
        self.experts = experts
        self.config = config if config is not None else KernelConfig.named("128x64x32")
        dummy = _placeholder(a.device)
        layout = MoeLayout(
            experts=experts, n=n, k=k,
            a=a.data_ptr() or dummy, lda=_row_stride(a),
            b=b.data_ptr() or dummy, ldb=b.stride(1) if k > 1 else max(1, n), stride_b=b.stride(0) if experts > 1 else 0,
            c=(c.data_ptr() or dummy) if c is not None else None, ldc=_row_stride(c) if c is not None else max(1, n),
            d=d.data_ptr() or dummy, ldd=_row_stride(d), alpha=float(alpha), beta=float(beta), max_rows=rows)
        self._tensors = (a, b, c, d)
        with torch.cuda.device(self.device):
            self.moe = MoeGroupedGemm(layout, self.config, int(sort_mode))

    @property
    def output(self) -> torch.Tensor:
        return self._tensors[3]

    def run(self, counts: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        if counts.dtype != torch.int32 or counts.device != self.device or counts.numel() != self.experts:
            raise ValueError(f"counts must be int32 [{self.experts}] on {self.device}")
        if not counts.is_contiguous():
            raise ValueError("counts must be contiguous")
        with torch.cuda.device(self.device):
            stream = stream if stream is not None else torch.cuda.current_stream(self.device)
            _lib.check(self.moe.run(counts.data_ptr(), stream), "MoeGroupedGemm.run")
        return self.output

    def status(self) -> int:
        """Status bits of the last run (GGK_MOE_NEGATIVE, GGK_MOE_CLAMPED); reads device memory,
        so it waits for the run."""
        header = self.moe.device_buffers()[3]
        out = torch.empty(_lib.GGK_MOE_HEADER_INTS, dtype=torch.int32)
        torch.cuda.synchronize(self.device)
        _lib.check(_lib.lib().ggk_copy_to_host(out.data_ptr(), header, out.numel() * 4), "copy header")
        return int(out[_lib.GGK_MOE_STATUS])

    def close(self) -> None:
        self.moe.close()


# ---------------------------------------------------------------- custom op

@torch.library.custom_op(_OP_NAME, mutates_args=())
def _grouped_gemm_op(a: list[torch.Tensor], b: list[torch.Tensor], c: list[Optional[torch.Tensor]],
                     alpha: list[float], beta: list[float], sort_mode: int) -> list[torch.Tensor]:
    """c: one entry per problem (None where C is not read), or an empty list for no C at all."""
    return run_grouped_gemm(a, b, c if len(c) else None, alpha, beta, sort_mode=sort_mode)


@_grouped_gemm_op.register_fake
def _grouped_gemm_fake(a, b, c, alpha, beta, sort_mode):
    return [ai.new_empty((ai.shape[0], bi.shape[1]), dtype=torch.float32) for ai, bi in zip(a, b)]


grouped_gemm_op = _grouped_gemm_op
