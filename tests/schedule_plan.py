"""The executor's work-tile schedule, restated for the tests (not collected: no test_ prefix).

plan_schedule in csrc/grouped_gemm.cpp plans it on the host; moe_prepare_kernel in csrc/gg_moe.hip
plans the same one on the device.  It is this library's own load-balancing heuristic (the
reference claims tiles from one counter in tile order), so it has no reference counterpart; D does
not depend on it."""
import math

from grouped_gemm_gpu_kernel_amd import _lib


def plan_schedule(shapes, work, bm, bn, bk, reads_c):
    """The host build's schedule (plan_schedule, csrc/grouped_gemm.cpp) for problems in sorted order:
    shapes[i] = (m, n, k), work[i] work tiles of bm x bn, reads_c a bool or one per problem.  Estimated time of a problem in hundredths
    of a cycle: sum over its tm x tn work tiles of 150 + stages (31 + 0.029 (rows + cols)) +
    0.0023 rows cols (x2 with C), i.e. 1500000 W + stages (310000 W + 290 (m tn + n tm)) + 23 m n (46
    with C), each operation rounded in double, then taken as an integer clamped to 2^52.  One share
    is the total over the 8 chunks, rounded up.  Problems above one share (oversized) are cut across
    chunks when whole placement (longest first, each to the first least-loaded chunk) would leave
    more than a quarter of the total to stealing (the sum over chunks of their shortfall below one
    share): they run first, back to back, longest first (stable), and chunk boundary c (c = 1, ...)
    falls at the work tile nearest to where the run's time reaches c shares (within problem i, tile
    floor((c share - time before i) / total_i * work_i + 0.5), clamped to [0, work_i]); the chunk
    holding the run's end starts with the remainder as its load.  The other problems go whole,
    longest first (stable), to the first least-loaded chunk from that one on (integer loads); within
    a chunk, after the run's remainder, longest work tile (unclamped time / W) first, then position.
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
    int64_max = (1 << 63) - 1
    whole_sum = min(sum(total), int64_max)  # the host's sum saturates
    share = -(-whole_sum // chunks)
    by_total = sorted(range(count), key=lambda i: -total[i])
    oversized = 0
    while oversized < count and total[by_total[oversized]] > share:
        oversized += 1
    if oversized:
        whole = [0] * chunks
        for i in by_total:
            c = min(range(chunks), key=lambda d: whole[d])
            whole[c] = min(whole[c] + total[i], int64_max)
        stolen = sum(float(share - x) for x in whole if x < share)
        if stolen * 4.0 <= float(whole_sum):
            oversized = 0
    order, offsets, bounds = [], [0], [0] * (chunks + 1)
    load = [0] * chunks
    first = 0
    if oversized:
        run_time, c = 0, 1
        for i in by_total[:oversized]:
            while c < chunks and c * share < run_time + total[i]:
                x = float(c * share - run_time) / float(total[i]) * work[i]
                bounds[c] = offsets[-1] + min(max(int(math.floor(x + 0.5)), 0), work[i])
                c += 1
            order.append(i)
            offsets.append(offsets[-1] + work[i])
            run_time += total[i]
        first = c - 1
        load[first] = run_time - first * share
    members = [[] for _ in range(chunks)]
    for i in by_total[oversized:]:
        c = min(range(first, chunks), key=lambda d: load[d])  # the first least-loaded chunk
        load[c] = min(load[c] + total[i], int64_max)
        members[c].append(i)
    for c in range(first, chunks):
        for i in sorted(members[c], key=lambda i: (-key[i], i)):
            order.append(i)
            offsets.append(offsets[-1] + work[i])
        bounds[c + 1] = offsets[-1]
    return order, offsets, bounds
