"""The C-ABI library loads and exports every function include/*.h declares (no GPU calls), and the
ctypes binding covers each of them."""
import re
import subprocess
from pathlib import Path

from grouped_gemm_gpu_kernel_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADERS = [ROOT / "include" / "grouped_gemm_amd.h", ROOT / "include" / "grouped_gemm_amd_kernels.h"]
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*\b((?:gg|ggk)_[a-z0-9_]+)\s*\(", re.M)


def declared_functions():
    names = set()
    for h in HEADERS:
        names |= set(DECL.findall(h.read_text()))
    return names


def test_headers_declare_the_api():
    names = declared_functions()
    for required in ("gg_prepare_problem_set", "gg_executor_build", "gg_executor_run", "gg_query_occupancy",
                     "gg_run_baseline_per_problem", "gg_run_grouped_gemm_once", "ggk_launch_grouped",
                     "ggk_launch_single", "ggk_kernel_resources_get", "ggk_occupancy"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared_functions() <= exported


def test_binding_covers_every_declared_symbol():
    assert declared_functions() == set(_lib.SIGNATURES)


def test_library_links_hip_and_has_gfx950_code():
    out = subprocess.run(["ldd", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    assert "libamdhip64" in out
    blob = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in blob


def test_cpp_api_header_mirrors_reference_names():
    text = (ROOT / "include" / "grouped_gemm" / "grouped_gemm.h").read_text()
    for name in ("enum class SortMode", "struct ProblemDesc", "struct KernelConfig", "struct PreparedProblemSet",
                 "struct OccupancyInfo", "class GroupedGemmExecutor", "prepare_problem_set(", "sort_mode_name(",
                 "query_occupancy(", "run_grouped_gemm_once(", "run_baseline_per_problem(",
                 "count_non_empty_problems(", "DeviceProblemDesc"):
        assert name in text, name


def test_addressing_form_classifier():
    """ggk_needs_addr64 (host-only) picks 64-bit addressing exactly when a problem's tile offsets would
    not stay below 2^31 bytes: work-tile rows * lda + K + 8 * stage_k >= 2^30 or stage_k * ldb >= 2^30
    (binary16 elements), rows * ldd + cols >= 2^29 or, when C is read, rows * ldc + cols >= 2^29 (float
    elements), or a negative leading dimension."""
    lib = _lib.lib()
    shape = _lib.GGKWorkShape()

    def needs(variant, path, lda, ldb, tiles=1, ldc=1, ldd=1, c=None, beta=0.0):
        p = _lib.GGDeviceProblemDesc(m=1, n=1, k=1, c=c, lda=lda, ldb=ldb, ldc=ldc, ldd=ldd, beta=beta,
                                     tiles_m=tiles, tiles_n=tiles)
        return lib.ggk_needs_addr64(variant, path, p)

    for variant, cta_m, cta_n in ((_lib.GGK_VARIANT_64x64x16, 64, 64), (_lib.GGK_VARIANT_128x64x32, 128, 64),
                                  (_lib.GGK_VARIANT_64x128x32, 64, 128), (_lib.GGK_VARIANT_128x64x32_SMALL, 128, 64),
                                  (_lib.GGK_VARIANT_64x128x32_SMALL, 64, 128),
                                  (_lib.GGK_VARIANT_64x64x16_SMALL, 64, 64)):
        for path in (_lib.GGK_PATH_FMA, _lib.GGK_PATH_MFMA):
            assert lib.ggk_work_shape_get(variant, path, shape) == 0
            assert shape.rows == cta_m * shape.tiles_m and shape.stage_k in (32, 64)
            # smallest lda that does not fit, for K = 1
            limit_a = ((1 << 30) - 2 - 8 * shape.stage_k) // shape.rows + 1
            limit_b = (1 << 30) // shape.stage_k
            assert needs(variant, path, limit_a - 1, 8) == 0
            assert needs(variant, path, limit_a, 8) == 1
            assert needs(variant, path, 8, limit_b - 1) == 0
            assert needs(variant, path, 8, limit_b) == 1
            assert needs(variant, path, -1, 8) == 1 and needs(variant, path, 8, -1) == 1
            assert needs(variant, path, 1 << 30, 1 << 30, tiles=0) == 0  # no tiles, nothing addressed
            # smallest ldc / ldd that does not fit
            limit_out = ((1 << 29) - 1 - cta_n * shape.tiles_n) // shape.rows + 1
            assert needs(variant, path, 8, 8, ldd=limit_out - 1) == 0
            assert needs(variant, path, 8, 8, ldd=limit_out) == 1
            # ldc matters only when C is read
            assert needs(variant, path, 8, 8, ldc=limit_out) == 0
            assert needs(variant, path, 8, 8, ldc=limit_out, c=64, beta=0.0) == 0
            assert needs(variant, path, 8, 8, ldc=limit_out, c=64, beta=0.5) == 1
            assert needs(variant, path, 8, 8, ldc=limit_out - 1, c=64, beta=0.5) == 0
    assert lib.ggk_needs_addr64(7, 0, _lib.GGDeviceProblemDesc()) == -1
    # every configuration on 256 x 256 work tiles, eight waves
    for variant, want in ((_lib.GGK_VARIANT_128x64x32, (2, 4, 512, 256, 64)),
                          (_lib.GGK_VARIANT_64x64x16, (4, 4, 512, 256, 64)),
                          (_lib.GGK_VARIANT_64x128x32, (4, 2, 512, 256, 64)),
                          # the same macro-tiles on 128 x 128 work tiles, for launches with few work tiles
                          (_lib.GGK_VARIANT_128x64x32_SMALL, (1, 2, 256, 128, 64)),
                          (_lib.GGK_VARIANT_64x128x32_SMALL, (2, 1, 256, 128, 64)),
                          (_lib.GGK_VARIANT_64x64x16_SMALL, (2, 2, 256, 128, 64))):
        assert lib.ggk_work_shape_get(variant, _lib.GGK_PATH_MFMA, shape) == 0
        assert (shape.tiles_m, shape.tiles_n, shape.threads, shape.rows, shape.stage_k) == want, variant
        # the 256 x 256 forms list tail work tiles as row halves
        assert lib.ggk_work_halves_supported(variant, _lib.GGK_PATH_MFMA) == (1 if want[2] == 512 else 0)
    # each large form's 128 x 128 counterpart has the same macro-tile
    for variant, small in ((_lib.GGK_VARIANT_64x64x16, _lib.GGK_VARIANT_64x64x16_SMALL),
                           (_lib.GGK_VARIANT_128x64x32, _lib.GGK_VARIANT_128x64x32_SMALL),
                           (_lib.GGK_VARIANT_64x128x32, _lib.GGK_VARIANT_64x128x32_SMALL)):
        assert lib.ggk_small_variant(variant) == small
        big, little = _lib.GGKWorkShape(), _lib.GGKWorkShape()
        assert lib.ggk_work_shape_get(variant, _lib.GGK_PATH_MFMA, big) == 0
        assert lib.ggk_work_shape_get(small, _lib.GGK_PATH_MFMA, little) == 0
        assert big.rows // big.tiles_m == little.rows // little.tiles_m  # macro-tile rows
    for variant in (_lib.GGK_VARIANT_64x64x16_SMALL, _lib.GGK_VARIANT_128x64x32_SMALL,
                    _lib.GGK_VARIANT_64x128x32_SMALL, -1, 6):
        assert lib.ggk_small_variant(variant) == -1


def test_failed_build_blocks_run():
    """After a rejected build the executor refuses to launch (hipErrorInvalidValue) instead of running
    a half-configured set; a never-built executor runs nothing and succeeds, as in the reference.
    Unsupported configurations and unusable argument lists are rejected before any device call, so
    this runs without a GPU."""
    import ctypes

    lib = _lib.lib()
    ex = lib.gg_executor_create()
    try:
        assert lib.gg_executor_run(ex, None) == _lib.HIP_SUCCESS
        bad_cfg = _lib.GGKernelConfig(128, 64, 32, 128, 0, 1)  # threads must be 256
        probs = (_lib.GGProblemDesc * 1)(_lib.GGProblemDesc(4, 4, 4, 0x1000, 0x2000, None, 0x3000, 4, 4, 4, 4,
                                                            1.0, 0.0))
        offs = (ctypes.c_int * 2)(0, 1)
        assert lib.gg_executor_build(ex, probs, 1, offs, 2, 1, ctypes.byref(bad_cfg)) == _lib.HIP_ERROR_INVALID_VALUE
        assert lib.gg_executor_run(ex, None) == _lib.HIP_ERROR_INVALID_VALUE
        assert lib.gg_executor_run_traced(ex, None, None, None, None) == _lib.HIP_ERROR_INVALID_VALUE
        assert lib.gg_executor_launched_work_tiles(ex) == 0
        assert lib.gg_executor_total_tiles(ex) == 0 and lib.gg_executor_problem_count(ex) == 0
        # a NULL problem list with a non-zero count and a NULL config are rejected the same way
        assert lib.gg_executor_build(ex, None, 3, offs, 2, 1, ctypes.byref(bad_cfg)) != _lib.HIP_SUCCESS
        assert lib.gg_executor_run(ex, None) == _lib.HIP_ERROR_INVALID_VALUE
        assert lib.gg_executor_build(ex, probs, 1, offs, 2, 1, None) != _lib.HIP_SUCCESS
        assert lib.gg_executor_run(ex, None) == _lib.HIP_ERROR_INVALID_VALUE
    finally:
        lib.gg_executor_destroy(ex)


def _gfx950_disassembly(tmp_path) -> str:
    """AMD assembly of the library's first gfx950 code object (the GEMM kernels), from its
    .hip_fatbin section."""
    llvm = Path("/opt/rocm/llvm/bin")
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([str(llvm / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", str(_lib.LIB_PATH),
                    str(tmp_path / "copy.so")], check=True, capture_output=True)
    code = tmp_path / "gfx950.o"
    subprocess.run([str(llvm / "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={fatbin}", f"--output={code}"],
                   check=True, capture_output=True)
    return subprocess.run([str(llvm / "llvm-objdump"), "-d", "--mcpu=gfx950", str(code)], check=True,
                          capture_output=True, text=True).stdout


def test_lds_loads_carry_their_wait_states(tmp_path):
    """The global -> LDS loads are inline assembly, which the compiler's hazard pass does not treat as
    memory instructions, so each must bring its own wait states: a VALU write of an SGPR the load
    reads (offset, resource words; v_readfirstlane right before the statement) needs 5, a SALU write
    of M0 needs 1.  Every `buffer_load_dwordx4 ... lds` of the built code must directly follow
    `s_nop N` with N >= 4 (N + 1 wait states)."""
    dis = _gfx950_disassembly(tmp_path)
    ins = [ln.split("//")[0].strip() for ln in dis.splitlines() if ln.startswith("\t")]
    ins = [x for x in ins if x]
    loads = [i for i, x in enumerate(ins) if x.startswith("buffer_load_dwordx4") and x.endswith(" lds")]
    assert len(loads) > 100, "expected the LDS-DMA loads of the MFMA kernels"
    bad = []
    for i in loads:
        prev = ins[i - 1].split()
        if not (prev[0] == "s_nop" and int(prev[1], 0) >= 4):
            bad.append(ins[i - 3:i + 1])
    assert not bad, f"{len(bad)} LDS loads without wait states, e.g. {bad[0]}"
