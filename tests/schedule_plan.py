"""The executor's work-tile schedule and launch plan, restated for the tests (not collected: no
test_ prefix).

plan_schedule in csrc/grouped_gemm.cpp plans the schedule on the host; moe_prepare_kernel in
csrc/gg_moe.hip plans the same one on the device.  plan_launch (csrc/grouped_gemm.cpp) adds the
variant choice, the grid and the work table with its tail halves.  All of it is this library's
own load balancing (the reference claims tiles from one counter in tile order), so it has no
reference counterpart; D does not depend on it."""
import heapq
import math

from grouped_gemm_gpu_kernel_amd import _lib


def problem_times(shapes, work, bm, bn, bk, reads_c):
    """Per problem: the estimated time the schedule ranks (an integer, clamped to 2^52) and the
    estimated time of one of its work tiles (unclamped time / work tiles); see plan_schedule."""
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
    return total, key


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
    total, key = problem_times(shapes, work, bm, bn, bk, reads_c)
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


# The work table's tail halves (GroupedGemmExecutor::build, csrc/grouped_gemm.cpp).
TAIL_HALVES = 64              # last work tiles of each chunk that may be listed as halves
TAIL_HALVES_MAX_PER_SLOT = 12  # only for sets of at most this many work tiles per workgroup
TAIL_HALVES_MIN_IDLE = 0.02    # and whose planned schedule leaves at least this idle share
WORK_TABLE_MAX = 1 << 22       # larger sets have no work table (the kernel searches)
SMALL_SET_TILES_PER_CU = 4     # 128 x 128 work tiles per CU at or below which the small form runs


def planned_idle_share(offsets, bounds, tile_time, grid):
    """Idle share of a schedule at its end by the tile-time estimate: the work tiles of chunk c, in
    claim order, go to whichever of its (grid - 1 - c) // 8 + 1 workgroups is free first; the share
    is 1 - busy / (workgroups x the latest end).  tile_time[pos]: one work tile's time of the
    problem at scheduling position pos."""
    chunks = _lib.GGK_SCHEDULER_CHUNKS
    busy, longest, slots_total, pos = 0.0, 0.0, 0, 0
    for c in range(chunks):
        slots = (grid - 1 - c) // chunks + 1 if c < grid else 0
        ends = [0.0] * slots
        for t in range(bounds[c], bounds[c + 1] if slots else bounds[c]):
            while offsets[pos + 1] <= t:
                pos += 1
            heapq.heappush(ends, heapq.heappop(ends) + tile_time[pos])
            busy += tile_time[pos]
        longest = max([longest] + ends)
        slots_total += slots
    return 1.0 - busy / (slots_total * longest) if longest > 0.0 and slots_total > 0 else 0.0


def work_tile_row(local, wtm, wtn):
    """Row of work tiles of work tile `local` in the grouped kernel's order: groups of 4 rows,
    column by column within a group."""
    group = local // (4 * wtn)
    first = group * 4
    rows = min(4, wtm - first)
    return first + (local - group * 4 * wtn) % rows


def grid_for(total, persistent, compute_units, blocks):
    """grid_ctas_for over `total` claimable units."""
    if total <= 0:
        return 0
    grid = persistent if persistent > 0 else min(compute_units * max(1, blocks), max(total, compute_units))
    return max(1, grid)


def plan_launch(problems, cta, mfma, compute_units, blocks_per_cu, work_shape, halves_supported, needs_addr64):
    """GroupedGemmExecutor::build's launch plan for sorted problems (m, n, k, reads_c):
    cta = (cta_m, cta_n, persistent_ctas), base variant = cta's.  The small form (128 x 128 work
    tiles) runs when the set has at most 4 such work tiles per CU, or when the base form needs 64-bit
    addressing (needs_addr64(variant) -> bool for the whole set); work_shape(variant) -> (tiles_m,
    tiles_n, stage_k), halves_supported(variant) -> bool.  Then the schedule (plan_schedule), the grid
    over the work tiles, and the work table: (problem, work tile) pairs in claim order, where within
    the last 64 work tiles of each chunk a work tile with more than half its rows inside the problem
    is listed as two halves (1 << 28 and 2 << 28 over the local index) -- when halves are supported,
    the set has at most 12 work tiles per workgroup and the schedule's planned idle share is at least
    0.02.  Returns a dict with the fields of gg_launch_plan plus order, offsets and table."""
    base, small = cta["variant"], cta["small"]
    chunks = _lib.GGK_SCHEDULER_CHUNKS
    tiles = [((m - 1) // cta["m"] + 1, (n - 1) // cta["n"] + 1) if m > 0 and n > 0 else (0, 0)
             for (m, n, k, _) in problems]

    def works(v):
        tm, tn, _ = work_shape(v)
        return [(a + tm - 1) // tm * ((b + tn - 1) // tn) for a, b in tiles]

    variant = base
    if mfma and small is not None and sum(works(small)) <= SMALL_SET_TILES_PER_CU * compute_units:
        variant = small
    if needs_addr64(variant) and mfma and small is not None and variant == base:
        variant = small
    addressing = 1 if needs_addr64(variant) else 0
    tm, tn, bk = work_shape(variant)
    work = works(variant)
    bm, bn = cta["m"] * tm, cta["n"] * tn
    shapes = [(m, n, k) for (m, n, k, _) in problems]
    reads = [r for (_, _, _, r) in problems]
    order, offsets, bounds = plan_schedule(shapes, work, bm, bn, bk, reads)
    _, key = problem_times(shapes, work, bm, bn, bk, reads)
    total_work = offsets[-1]
    grid = grid_for(total_work, cta["persistent"], compute_units, blocks_per_cu[variant])
    table, launch, halves = [], list(bounds), False
    if 0 < total_work <= WORK_TABLE_MAX:
        halves = (halves_supported(variant) and total_work <= TAIL_HALVES_MAX_PER_SLOT * grid and
                  planned_idle_share(offsets, bounds, [key[i] for i in order], grid) >= TAIL_HALVES_MIN_IDLE)
        index, chunk, launch = 0, 0, [0] * (chunks + 1)
        for prob in order:
            wtm, wtn = (tiles[prob][0] + tm - 1) // tm, (tiles[prob][1] + tn - 1) // tn
            for w in range(work[prob]):
                while chunk < chunks and index >= bounds[chunk + 1]:
                    chunk += 1
                    launch[chunk] = len(table) // 2
                tail = halves and index >= bounds[chunk + 1] - TAIL_HALVES
                if tail and problems[prob][0] - work_tile_row(w, wtm, wtn) * bm > bm // 2:
                    table += [prob, w | (1 << 28), prob, w | (2 << 28)]
                else:
                    table += [prob, w]
                index += 1
        while chunk < chunks:
            chunk += 1
            launch[chunk] = len(table) // 2
    return dict(variant=variant, addressing=addressing, total_work=total_work,
                launch_total=len(table) // 2 if table else total_work, grid=grid, halves=halves, order=order,
                offsets=offsets, bounds=bounds, table=table, launch_bounds=launch)


def plan_shards(problems, ranks, bm, bn, bk):
    """grouped_gemm::plan_shards (csrc/grouped_gemm.cpp) for problems (m, n, k, reads_c): the
    estimate of a piece of `cols` columns is the schedule's model on bm x bn work tiles (unclamped
    double); a problem above one rank's share (total / ranks) is cut into min(work-tile columns,
    ceil(t / share)) column ranges, the first ones one work-tile column wider when they do not divide
    evenly; pieces go longest first (stable), each to the least-loaded rank (lowest on ties), an
    empty problem whole to rank 0.  Returns [(problem, rank, col0, cols)] in problem order."""
    def estimate(m, cols, k, reads_c):
        if m <= 0 or cols <= 0:
            return 0.0
        tm, tn = (m - 1) // bm + 1, (cols - 1) // bn + 1
        wt = float(tm) * tn
        stages = float((k - 1) // bk + 1) if k > 0 else 0.0
        edge = float(m) * tn + float(cols) * tm
        stage = 310000.0 * wt + 290.0 * edge
        return 1500000.0 * wt + stages * stage + (46.0 if reads_c else 23.0) * (float(m) * cols)

    total = 0.0
    for (m, n, k, c) in problems:
        total += estimate(m, n, k, c)
    share = total / ranks
    pieces, times = [], []
    for i, (m, n, k, c) in enumerate(problems):
        t = estimate(m, n, k, c)
        wtn = (n - 1) // bn + 1 if n > 0 else 0
        parts = 1
        if share > 0.0 and t > share and wtn > 1:
            parts = int(min(float(wtn), math.ceil(t / share)))
        first = 0
        for part in range(parts):
            span = wtn // parts + (1 if part < wtn % parts else 0)
            col0 = first * bn
            cols = n if parts == 1 else min(n - col0, span * bn)
            pieces.append([i, 0, col0, cols])
            times.append(t if parts == 1 else estimate(m, cols, k, c))
            first += span
    load = [0.0] * ranks
    for j in sorted(range(len(pieces)), key=lambda j: -times[j]):
        if times[j] <= 0.0:
            continue
        r = min(range(ranks), key=lambda x: load[x])
        pieces[j][1] = r
        load[r] += times[j]
    return [tuple(p) for p in pieces]
