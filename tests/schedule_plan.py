"""The executor's work-tile schedule, restated for the tests (not collected: no test_ prefix).

plan_schedule in csrc/grouped_gemm.cpp plans it on the host; moe_prepare_kernel in csrc/gg_moe.hip
plans the same one on the device.  It is this library's own load-balancing heuristic (the
reference claims tiles from one counter in tile order), so it has no reference counterpart; D does
not depend on it."""
from grouped_gemm_gpu_kernel_amd import _lib


def plan_schedule(shapes, work, bm, bn, bk, reads_c):
    """The host build's schedule (plan_schedule, csrc/grouped_gemm.cpp) for problems in sorted order:
    shapes[i] = (m, n, k), work[i] work tiles of bm x bn, reads_c a bool or one per problem.  Estimated time of a problem in hundredths
    of a cycle: sum over its tm x tn work tiles of 150 + stages (31 + 0.029 (rows + cols)) +
    0.0023 rows cols (x2 with C), i.e. 1500000 W + stages (310000 W + 290 (m tn + n tm)) + 23 m n (46
    with C), each operation rounded in double, then taken as an integer clamped to 2^52.  Problems go
    whole, longest first (stable), to the first least-loaded of the 8 chunks (integer loads); within
    a chunk, longest work tile (unclamped time / W) first, then position.
    Returns (order, work offsets in that order, chunk bounds)."""
    count = len(shapes)
    reads = list(reads_c) if isinstance(reads_c, (list, tuple)) else [bool(reads_c)] * count
    total, key = [0] * count, [0.0] * count
    for i, ((m, n, k), w) in enumerate(zip(shapes, work)):
        if w <= 0:
            continue
        tm, tn = (m - 1) // bm + 1, (n - 1) // bn + 1
        wt = float(tm) * tn
        stages = float((k - 1) // bk + 1) if k > 0 else 0.0
        edge = float(m) * tn + float(n) * tm
        stage = 310000.0 * wt + 290.0 * edge
        area = float(m) * n
        t = 1500000.0 * wt + stages * stage + (46.0 if reads[i] else 23.0) * area
        total[i] = int(t) if t < 2.0 ** 52 else 1 << 52
        key[i] = t / w
    chunks = _lib.GGK_SCHEDULER_CHUNKS
    load = [0] * chunks
    members = [[] for _ in range(chunks)]
    for i in sorted(range(count), key=lambda i: -total[i]):
        c = min(range(chunks), key=lambda d: load[d])  # the first least-loaded chunk
        load[c] += total[i]
        members[c].append(i)
    order, offsets, bounds = [], [0], [0]
    for c in range(chunks):
        for i in sorted(members[c], key=lambda i: (-key[i], i)):
            order.append(i)
            offsets.append(offsets[-1] + work[i])
        bounds.append(offsets[-1])
    return order, offsets, bounds
