"""The PyTorch binding (grouped_gemm_gpu_kernel_amd/torch_ops.py): argument checking and the fake
(shape) implementation on the CPU; on the GPU, results against the oracle's host GEMM
(tests/test_correctness.cu:85-102 restated) within 1e-3*sqrt(K)*max|A|*max|B|*|alpha| plus a few
float32 ulps of the beta*C term, plan reuse across streams, and the registered custom op."""
import math

import numpy as np
import pytest
import torch

from grouped_gemm_gpu_kernel_amd import torch_ops
from grouped_gemm_gpu_kernel_amd.api import KernelConfig, SortMode
from oracle import oracle as O


def tolerance(k, max_a, max_b, max_c, alpha, beta):
    return 1e-3 * math.sqrt(max(k, 1)) * max_a * max_b * abs(alpha) + 1e-6 * (abs(beta) * max_c + 1.0)


# ---------------------------------------------------------------- CPU

def test_rejects_host_tensors_and_mismatched_lists():
    a = [torch.zeros(4, 8, dtype=torch.float16)]
    b = [torch.zeros(8, 3, dtype=torch.float16)]
    with pytest.raises(ValueError, match="on a GPU"):
        torch_ops.run_grouped_gemm(a, b)
    with pytest.raises(ValueError, match="one tensor per problem"):
        torch_ops.run_grouped_gemm(a, b + b)
    with pytest.raises(ValueError, match="one tensor per problem"):
        torch_ops.GroupedGemmPlan(a, b, None, [])


def test_empty_problem_list():
    assert torch_ops.run_grouped_gemm([], []) == []


def test_empty_matrices_ignore_strides():
    """An empty matrix may carry any strides (numpy's (0, k) arrays do); its row stride is unused."""
    t = torch.from_numpy(np.zeros((0, 16), np.float16))
    torch_ops._check_matrix(t, "a", torch.float16, None, t.device)
    assert torch_ops._row_stride(t) == 16
    assert torch_ops._row_stride(torch.empty(5, 0)) == 1


def test_fake_implementation_gives_output_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        a = [torch.empty(5, 7, dtype=torch.float16), torch.empty(0, 3, dtype=torch.float16)]
        b = [torch.empty(7, 9, dtype=torch.float16), torch.empty(3, 4, dtype=torch.float16)]
        out = torch.ops.grouped_gemm_amd.grouped_gemm(a, b, [], [1.0, 1.0], [0.0, 0.0], int(SortMode.kByK))
        assert [tuple(t.shape) for t in out] == [(5, 9), (0, 4)]
        assert all(t.dtype == torch.float32 for t in out)


# ---------------------------------------------------------------- GPU

def _operands(shapes, seed, pad=0, c_every=1):
    """fp16 A/B uniform[-1, 1], fp32 C uniform[-1, 1]; with pad > 0 every A, B, C and D is a column
    slice of a wider tensor (row stride above the row length)."""
    rng = np.random.default_rng(seed)
    dev = torch.device("cuda")
    a, b, c, d, host = [], [], [], [], []
    for i, (m, n, k) in enumerate(shapes):
        ah = rng.uniform(-1, 1, (m, k)).astype(np.float16)
        bh = rng.uniform(-1, 1, (k, n)).astype(np.float16)
        ch = rng.uniform(-1, 1, (m, n)).astype(np.float32) if i % c_every == 0 else None

        def place(x, dtype):
            full = torch.zeros((x.shape[0], x.shape[1] + pad), dtype=dtype, device=dev)
            view = full[:, :x.shape[1]]
            view.copy_(torch.from_numpy(x))
            return view

        a.append(place(ah, torch.float16))
        b.append(place(bh, torch.float16))
        c.append(place(ch, torch.float32) if ch is not None else None)
        d.append(torch.full((m, n + pad), float("nan"), dtype=torch.float32, device=dev)[:, :n])
        host.append((ah, bh, ch))
    return a, b, c, d, host


def _check(shapes, host, d, alpha, beta):
    for i, ((m, n, k), (ah, bh, ch)) in enumerate(zip(shapes, host)):
        al = alpha[i] if isinstance(alpha, list) else alpha
        be = beta[i] if isinstance(beta, list) else beta
        want = O.gemm(m, n, k, ah.view(np.uint16), max(1, k), bh.view(np.uint16), max(1, n),
                      ch, max(1, n), al, be)[:m * n].reshape(m, n)
        got = d[i].cpu().numpy()
        assert not np.isnan(got).any(), i
        max_c = float(np.abs(ch).max()) if ch is not None and ch.size else 0.0
        err = float(np.abs(got - want).max()) if got.size else 0.0
        assert err <= tolerance(k, 1.0, 1.0, max_c, al, be), (i, (m, n, k), err)


SHAPES = [(64, 64, 64), (45, 81, 37), (1, 1, 1), (130, 17, 300), (0, 32, 16), (32, 0, 16), (17, 33, 0),
          (256, 200, 64), (7, 513, 9), (300, 64, 1000)]


@pytest.mark.gpu
@pytest.mark.parametrize("config", ["64x64x16", "128x64x32", "64x128x32"])
@pytest.mark.parametrize("mode", list(SortMode))
def test_run_grouped_gemm_matches_oracle(torch_cuda, config, mode):
    alpha = [0.5 + 0.25 * i for i in range(len(SHAPES))]
    beta = [0.0 if i % 4 == 3 else 0.125 * i for i in range(len(SHAPES))]
    a, b, c, d, host = _operands(SHAPES, seed=int(mode) * 7 + len(config), pad=3 if int(mode) % 2 else 0, c_every=2)
    out = torch_ops.run_grouped_gemm(a, b, c, alpha, beta, sort_mode=mode, config=KernelConfig.named(config),
                                     out=d)
    assert all(o is di for o, di in zip(out, d))
    _check(SHAPES, host, d, alpha, [be if ci is not None else 0.0 for be, ci in zip(beta, c)])


@pytest.mark.gpu
def test_allocates_outputs_and_fma_path(torch_cuda):
    a, b, c, _, host = _operands(SHAPES, seed=5)
    out = torch_ops.run_grouped_gemm(a, b, c, 2.0, 1.0,
                                     config=KernelConfig.named("64x64x16", use_tensor_cores=False))
    assert [tuple(o.shape) for o in out] == [(m, n) for m, n, _ in SHAPES]
    assert all(o.dtype == torch.float32 and o.is_contiguous() for o in out)
    _check(SHAPES, host, out, 2.0, 1.0)


@pytest.mark.gpu
def test_plan_reruns_on_side_stream_after_inputs_change(torch_cuda):
    a, b, c, d, host = _operands(SHAPES, seed=9)
    plan = torch_ops.GroupedGemmPlan(a, b, c, d, 1.0, 0.5, sort_mode=SortMode.kByTiles)
    plan.run()
    torch.cuda.synchronize()
    _check(SHAPES, host, d, 1.0, 0.5)
    rng = np.random.default_rng(10)
    side = torch.cuda.Stream()
    new_host = []
    for i, (ah, bh, ch) in enumerate(host):
        ah2 = rng.uniform(-1, 1, ah.shape).astype(np.float16)
        a[i].copy_(torch.from_numpy(ah2))
        new_host.append((ah2, bh, ch))
    side.wait_stream(torch.cuda.current_stream())
    for _ in range(3):
        plan.run(side)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _check(SHAPES, new_host, d, 1.0, 0.5)
    plan.close()


@pytest.mark.gpu
def test_custom_op(torch_cuda):
    a, b, c, _, host = _operands(SHAPES[:4], seed=13, c_every=2)
    out = torch.ops.grouped_gemm_amd.grouped_gemm(a, b, c, [1.0] * 4, [1.0] * 4, int(SortMode.kByK))
    _check(SHAPES[:4], host, out, 1.0, 1.0)
    out = torch.ops.grouped_gemm_amd.grouped_gemm(a, b, [], [1.5] * 4, [1.0] * 4, int(SortMode.kNone))
    _check(SHAPES[:4], [(ah, bh, None) for ah, bh, _ in host], out, 1.5, 0.0)


@pytest.mark.gpu
def test_argument_errors_on_gpu_tensors(torch_cuda):
    dev = torch.device("cuda")
    a = [torch.zeros(4, 8, dtype=torch.float16, device=dev)]
    b = [torch.zeros(8, 3, dtype=torch.float16, device=dev)]
    with pytest.raises(TypeError, match="float16"):
        torch_ops.run_grouped_gemm([a[0].float()], b)
    with pytest.raises(ValueError, match="rows"):
        torch_ops.run_grouped_gemm(a, [torch.zeros(7, 3, dtype=torch.float16, device=dev)])
    with pytest.raises(ValueError, match="contiguous rows"):
        torch_ops.run_grouped_gemm([torch.zeros(8, 4, dtype=torch.float16, device=dev).t()], b)
    with pytest.raises(ValueError, match="shape"):
        torch_ops.run_grouped_gemm(a, b, [torch.zeros(4, 4, device=dev)])
    with pytest.raises(ValueError, match="entries"):
        torch_ops.run_grouped_gemm(a, b, None, [1.0, 2.0])
