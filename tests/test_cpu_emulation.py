"""libaffx's kernels run on the CPU (tests/cpu_emu): every launch emulated with one thread per
work-item, real barriers, exact MFMA, under AddressSanitizer. Checks bounds of every device
access and the numerics against the oracle, without a GPU. Sizes are kept small: the emulation
runs each work-item as an OS thread."""
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang"
CLANGXX = "/opt/rocm/llvm/bin/clang++"


# the library sources the emulator links, each its own translation unit as in the device build
SOURCES = ["affx_layout.hip", "affx_decode.hip", "affx_fused.hip", "affx_quant.hip", "affx_grouped.hip",
           "affx_api.hip", "affx_noalloc.hip", "affx_route.hip", "affx_shared.hip", "affx_fit.hip", "affx_gemv.hip",
           "affx_steps.hip", "affx_w8a8.hip"]


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    if not (os.path.exists(CLANGXX) and os.path.exists(CLANG)):
        pytest.skip("clang++ not available")
    d = tmp_path_factory.mktemp("emu")
    san = ["-fsanitize=address", "-fno-omit-frame-pointer", "-g", "-O1"]
    # -ffp-contract=fast-honor-pragmas with FMA available mirrors the device compiler's default
    # for HIP, so a kernel that needs exact float order has to say so itself (a contract pragma)
    cxx = [CLANGXX, "-std=c++20", *san, "-march=x86-64-v3", "-ffp-contract=fast-honor-pragmas", "-w",
           "-I", os.path.join(ROOT, "tests", "cpu_emu"), "-I", os.path.join(ROOT, "affinity_amd", "csrc")]
    jobs = [[CLANG, *san, "-ffp-contract=off", "-fopenmp=libgomp", "-c",
             os.path.join(ROOT, "oracle", "oracle.c"), "-o", str(d / "oracle.o")],
            [*cxx, "-c", os.path.join(ROOT, "tests", "cpu_emu", "emu_main.cpp"), "-o", str(d / "emu_main.o")]]
    objs = [str(d / "oracle.o"), str(d / "emu_main.o")]
    for src in SOURCES:
        o = str(d / (src + ".o"))
        jobs.append([*cxx, "-x", "c++", "-c", os.path.join(ROOT, "affinity_amd", "csrc", src), "-o", o])
        objs.append(o)
    with ThreadPoolExecutor(max_workers=8) as pool:
        for r in pool.map(lambda cmd: subprocess.run(cmd, capture_output=True, text=True), jobs):
            assert r.returncode == 0, r.stderr[-4000:]
    subprocess.run([CLANGXX, *san, *objs, "-o", str(d / "emu_main"), "-lpthread", "-fopenmp=libgomp"], check=True)
    return str(d / "emu_main")


def run(emu, *args, timeout=900, cus=4):
    # cus: compute units of the emulated device; the fused decode sizes its grid (all workgroups
    # resident, run concurrently here) to it
    # (a generous bound on the decode's waits: an emulated waiter polls with a thread yield, and
    # on a loaded host 2^22 yields can pass before the emulated workgroups it waits for are done)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", AFFX_EMU_CUS=str(cus),
               AFFX_DECODE_SPIN_LIMIT=str(1 << 30))
    r = subprocess.run([emu, *map(str, args)], cwd=ROOT, capture_output=True, text=True,
                       timeout=timeout, env=env)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    return out


# Every case's arguments (and emulated CU count). The runs are started together, three at a time,
# when the first test asks for one: each is a long single-threaded-per-lane emulation, and
# running them side by side keeps the module's wall time near the longest few.
CASES = {
    "dequant": (("dequant", 1024, 1024, 1), 4),
    # decode: the fused launch is checked bit-identical to the staged launches, its counters zero
    # after two launches on one workspace, and both against the oracle at 1e-3 relative L2
    "decode_m1": (("decode", 1024, 1024, 7, 1, 6, 1), 4),   # 4 workgroups: gate/up in rounds
    "decode_allpad": (("decode", 1024, 1024, 5, 2, 3, 4, "allpad"), 3),
    "decode_m1_single": (("decode", 1024, 1024, 5, 1, 1, 9), 6),
    "decode_m6": (("decode", 2048, 1024, 5, 6, 2, 2), 4),
    "decode_m6_dm16": (("decode", 2048, 1024, 5, 6, 2, 2, "dm16"), 4),
    "decode_m8_wide": (("decode", 1024, 1024, 7, 8, 3, 6), 3),
    # three experts, every token routed to all three (token 0's last route padding): every slot
    # serves seven or eight tokens, so each one takes two passes of the compacted column group
    "decode_m8_full": (("decode", 1024, 1024, 3, 8, 3, 7), 3),
    "quant": (("quant", 4, 256, 3), 4),
    "grouped": (("grouped", 1024, 1024, 5, 12, 3, 4, 1), 4),
    "timeout": (("timeout", 1024, 1024, 6, 2, 3, 8), 4),
    # batch 1 in one pass (6 workgroups hold the 64 gate/up items): per-workgroup publish flags
    "timeout_m1": (("timeout", 1024, 1024, 6, 1, 1, 8), 6),
    "slots": (("slots", 1024, 1024, 4, 6, 2, 9), 4),
    "ffnptr": (("ffnptr", 1024, 1024, 3, 12), 4),
    # one expert at hidden 4096, inter 1024: the smallest scratch the reference's contract gives
    "ffnptr_n1": (("ffnptr", 4096, 1024, 1, 13), 4),
    "route": (("route", 21, 100, 6, 4), 4),
    # the single-matrix GEMV entries: 3 down matrices (1024 x 2048) in one batch, one alone
    "gemv": (("gemv", 1024, 2048, 3, 5), 4),
    # gather / scatter / SwiGLU requantise against the oracle (bounds checked)
    "steps": (("steps", 256, 40, 3), 4),
    # the single-matrix W8A8 GEMM: three tiles of down matrices (f32, strided arena, pad), one bf16
    "w8a8": (("w8a8", 1024, 1024, 7), 4),
    "shared": (("shared", 1024, 1024, 6, 40, 5), 4),
}
# longest first, so the three lanes finish together
ORDER = ["decode_m8_wide", "decode_m8_full", "decode_m6_dm16", "decode_m6", "slots", "shared", "decode_m1_single", "grouped",
         "decode_m1", "ffnptr", "ffnptr_n1", "quant", "timeout", "timeout_m1", "route", "gemv", "w8a8", "steps", "decode_allpad",
         "dequant"]


@pytest.fixture(scope="module")
def runs(emu):
    pool = ThreadPoolExecutor(max_workers=3)
    futs = {name: pool.submit(run, emu, *CASES[name][0], cus=CASES[name][1]) for name in ORDER}
    yield futs
    for f in futs.values():
        f.cancel()
    pool.shutdown(wait=True)


def result(runs, name):
    return runs[name].result()


def test_dequant_emulated(runs):
    assert "exact=1" in result(runs, "dequant")


def test_decode_emulated_m1(runs):
    # 4 workgroups: gate/up in rounds, several output tiles per workgroup
    assert "identical to staged=1" in result(runs, "decode_m1")


def test_decode_emulated_all_padding(runs):
    # no route names an expert of the layer: nothing to wait for, y written as zeros
    out = result(runs, "decode_allpad")
    assert "identical to staged=1" in out and "rel_l2=0.000e+00" in out


def test_decode_emulated_m1_single_pass(runs):
    # 6 workgroups hold all 64 gate/up items: the straight-line batch-1 variant
    assert "identical to staged=1" in result(runs, "decode_m1_single")


def test_decode_emulated_m6_compacted_columns(runs):
    # six tokens: each slot's tokens fill the one column group of the fused kernel in order (the
    # staged launches keep two fixed groups of five tokens)
    assert "identical to staged=1" in result(runs, "decode_m6")


def test_decode_emulated_m6_dim_major_arena(runs):
    # the engine's dim-major batch arena at its 16-token stride: whole-row reads of four tokens
    # per wave (two token quads x two column segments), the second quad half padding slots
    assert "identical to staged=1" in result(runs, "decode_m6_dm16")


def test_decode_emulated_m8_wide_epilogue(runs):
    # 12 gate/up groups x 16 rows x 8 tokens: the epilogue takes two passes of the workgroup
    # (hidden 1024: one column segment, so 12 wave groups; inter 1024 keeps the emulation short)
    assert "identical to staged=1" in result(runs, "decode_m8_wide")


def test_decode_emulated_m8_two_passes(runs):
    # every slot serves more than five tokens: a second pass over the same weight registers, and
    # the down phase's per-token sums across both passes
    assert "identical to staged=1" in result(runs, "decode_m8_full")


def test_quantizer_emulated(runs):
    assert "exact=1" in result(runs, "quant")


def test_grouped_emulated(runs):
    assert "rel_l2" in result(runs, "grouped")


def test_decode_wait_give_up_fails_loudly(runs):
    # the host forces the bounded wait to give up (no polls); the hook returns 0 with an error,
    # affx_decode_status reports it, and after the reset the next call is right
    out = result(runs, "timeout")
    assert "timeout path ok=1" in out, out


def test_decode_wait_give_up_fails_loudly_batch1(runs):
    # the same on the one-pass batch-1 kernel, whose waiters poll every workgroup's publish flag:
    # the give-up is reported, the reset clears the epoch and the flags, the next call is right
    out = result(runs, "timeout_m1")
    assert "timeout path ok=1" in out, out


def test_grouped_slot_list_emulated(runs):
    # the slot-list entry: bit-identical to the routes entry on the list the routes build, and
    # within tolerance on a reordered list
    out = result(runs, "slots")
    assert "routes==slots=1" in out, out


def test_expert_ffn_pointer_table_emulated(runs):
    out = result(runs, "ffnptr")
    assert "identical to staged=1" in out, out


def test_expert_ffn_pointer_table_one_expert_emulated(runs):
    out = result(runs, "ffnptr_n1")
    assert "ffnptr rc=0 identical to staged=1" in out, out


def test_gemv_emulated(runs):
    out = result(runs, "gemv")
    assert "gemv rc=0" in out, out


def test_w8a8_gemm_emulated(runs):
    """affx_expert_gemm_w8a8 within 1e-5 of the oracle (f32 outputs) and 1 bf16 ulp (bf16 output),
    the strided arena's other columns untouched."""
    out = result(runs, "w8a8")
    assert "w8a8 rc=0" in out and "others_kept=1" in out, out


def test_separable_steps_emulated(runs):
    out = result(runs, "steps")
    assert "equal=1" in out, out


def test_route_emulated(runs):
    out = result(runs, "route")
    assert "route ids equal=1" in out, out


def test_shared_expert_and_hc_post_emulated(runs):
    """The shared expert's decode (1 token; 3 tokens read dim-major; 6 tokens, two column groups)
    and batch kernels (40 tokens, with and without a low part) against the oracle, the
    hyper-connection post bit for bit."""
    out = result(runs, "shared")
    assert "shared ok=1" in out, out
