"""Register, scratch and LDS budgets of the kernel library, read from its gfx950 assembly.

A kernel that spills to scratch memory or whose LDS footprint grows past what its design
assumes still computes the right numbers, so no parity test notices; but on MI355X a GEMM
whose LDS grew by a promoted per-thread slot ran three times slower per launch. These checks
compile every csrc/*.hip for the device only (hipcc -S, no GPU needed) and read each kernel's
.amdhsa descriptor: no scratch (apart from the generic element-wise interpreter, whose register
file is indexed at run time), LDS within the CU's 160 KB, and the GEMM kernels' LDS exactly
their DMA rings.
"""

from __future__ import annotations

import re
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from ml_graph_compiler.codegen import build as native

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "ml-graph-compiler_amd" / "csrc"
LDS_PER_CU = 160 * 1024
# run-time indexed register files: the generic element-wise program and Range interpreters
SCRATCH_ALLOWED = ("ew_program_kernel", "range_kernel")


def _kernels(src: Path, out_dir: Path) -> dict[str, dict[str, int]]:
    asm = out_dir / (src.stem + ".s")
    cmd = [native.find_hipcc(), *native.HIPCC_FLAGS, "-S", "--cuda-device-only", "-I", str(ROOT / "include"),
           "-I", str(CSRC), str(src), "-o", str(asm)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    found: dict[str, dict[str, int]] = {}
    name = None
    for line in asm.read_text().splitlines():
        m = re.match(r"\s*\.amdhsa_kernel\s+(\S+)", line)
        if m:
            name = m.group(1)
            found[name] = {}
            continue
        m = re.match(r"\s*\.amdhsa_(private_segment_fixed_size|group_segment_fixed_size|next_free_vgpr)\s+(\d+)", line)
        if m and name:
            found[name][m.group(1)] = int(m.group(2))
    return found


@pytest.fixture(scope="module")
def kernels(tmp_path_factory) -> dict[str, dict[str, int]]:
    out = tmp_path_factory.mktemp("asm")
    sources = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=4) as pool:
        parts = list(pool.map(lambda s: _kernels(s, out), sources))
    merged: dict[str, dict[str, int]] = {}
    for p in parts:
        merged.update(p)
    return merged


def test_no_kernel_spills_to_scratch(kernels):
    spilled = {k: v["private_segment_fixed_size"] for k, v in kernels.items()
               if v.get("private_segment_fixed_size", 0) and not any(a in k for a in SCRATCH_ALLOWED)}
    assert not spilled, spilled
    assert len(kernels) > 40


def test_lds_fits_a_cu(kernels):
    over = {k: v["group_segment_fixed_size"] for k, v in kernels.items()
            if v.get("group_segment_fixed_size", 0) > LDS_PER_CU}
    assert not over, over


def test_gemm_lds_is_the_dma_rings(kernels):
    """32 x 32 wave split: 4 waves x 2 stages x (A + B) 32 x 32 floats = 64 KB; 16 x 16 wave split
    with S stages and W waves: W x S x 2 x 16 x 32 floats."""
    def lds(pattern: str) -> set[int]:
        return {v["group_segment_fixed_size"] for k, v in kernels.items() if re.search(pattern, k)}

    assert lds(r"gemm_dma_wsplit_kernel") == {65536}
    # 64 x 64 tiles, with and without the quarter-tile tail: a two-stage ring of 2 x 64 x 32 floats
    assert lds(r"gemm_dma_kernelILi64ELi64E|gemm_dma_tail_kernel") == {32768}
    assert lds(r"gemm_dma_wsplit16_kernelILi\dELi3ELi8E") == {8 * 3 * 4096}
    assert lds(r"gemm_dma_wsplit16_kernelILi\dELi2ELi4E") == {4 * 2 * 4096}


# Kernels that declare no shared memory. The compiler may still move a per-thread array into
# LDS (one slot per thread); on MI355X such a kernel ran five times slower (an embedding gather
# whose four 16-byte chunks per lane went through LDS: 17 us against 3 us), so LDS here is a
# regression.
NO_LDS = ("ew_f32_kernel", "ew_program_kernel", "copy_kernel", "gather_kernel", "gather_rows16_kernel",
          "fill_kernel", "range_kernel", "layer_norm_rows", "softmax_rows", "softmax_strided",
          "gemm_splitk_reduce", "gemm_splitk_layer_norm", "gemm_stream_kernel", "pool_nhwc",
          "depthwise3x3_nhwc_vec4", "depthwise_nhwc", "space_to_depth_kernel", "reduce_generic",
          "reduce_mid_rows", "reduce_mid_strided", "argmax_kernel")


def test_no_lds_where_none_is_declared(kernels):
    hits = {k: v["group_segment_fixed_size"] for k, v in kernels.items()
            if any(re.search(r"\d" + n + r"[EI]", k) for n in NO_LDS)}
    assert len(hits) >= len(NO_LDS), sorted(hits)
    used = {k: lds for k, lds in hits.items() if lds}
    assert not used, used
