"""hip backend checks that need no GPU: code generation, the native builds, the exported C ABI,
error behaviour, and the kernel mixes the reference reports for its configs."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from ml_graph_compiler import builders
from ml_graph_compiler.codegen import build as native
from ml_graph_compiler.codegen.hip import HipEmitter, generate_hip, pack_b_nk
from ml_graph_compiler.errors import CodegenError, ModelImportError
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from helpers import f32, op_graph

ROOT = Path(__file__).resolve().parents[1]


def declared_functions(header: Path) -> set[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set()
    for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mgc_\w+)\s*\(", text, flags=re.M):
        names.add(m.group(1))
    return names


def exported(lib: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def o3(graph):
    optimize(graph, "O3")
    schedule(graph)
    return graph


def test_kernel_library_exports_every_declared_symbol():
    lib = native.kernel_library_path()
    declared = declared_functions(ROOT / "include" / "mgc_hip.h")
    assert {"mgc_hip_gemm", "mgc_hip_model_run", "mgc_hip_elementwise"} <= declared
    missing = declared - exported(lib)
    assert not missing, missing
    handle = native.load_kernel_library()
    assert handle.mgc_hip_version().startswith(b"mgc_hip")
    assert handle.mgc_hip_device_count() >= 0


def test_ctypes_views_match_the_header_layout(tmp_path):
    """The ctypes structures the GPU tests pass to the C ABI (tests/capi.py and the entry-point
    tests' own mirrors) have the size and field offsets a C compiler gives the header's structs."""
    import ctypes

    import capi
    from test_gpu_conv_stem import ConvStemArgs, StemArgs
    from test_gpu_gather_layer_norm import GatherLnArgs
    from test_gpu_pool_fc import PoolFcArgs

    checks = [("mgc_hip_gemm_args", capi.GemmArgs), ("mgc_hip_operand", capi.Operand),
              ("mgc_hip_stem_args", StemArgs), ("mgc_hip_conv_stem_args", ConvStemArgs),
              ("mgc_hip_pool_fc_args", PoolFcArgs), ("mgc_hip_gather_ln_args", GatherLnArgs)]
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "mgc_hip.h"', "int main(void) {"]
    for cname, cls in checks:
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {tuple(line.split()[:2]): int(line.split()[2]) for line in out if line.strip()}
    for cname, cls in checks:
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert got[(cname, field)] == getattr(cls, field).offset, (cname, field)


def test_model_library_exports_the_model_abi(hip_cache):
    gen = generate_hip(o3(builders.mlp()), profile=True)
    built = native.build_model_library(gen.source, cache_dir=hip_cache, name="abi")
    declared = declared_functions(ROOT / "include" / "mgc_model.h")
    assert {"mgc_run", "mgc_arena_bytes", "mgc_weights_bytes", "mgc_hip_init", "mgc_profile_data"} <= declared
    missing = declared - exported(built.library)
    assert not missing, missing
    plain = native.build_model_library(generate_hip(o3(builders.mlp())).source, cache_dir=hip_cache, name="abi2")
    assert "mgc_profile_data" not in exported(plain.library)
    again = native.build_model_library(gen.source, cache_dir=hip_cache, name="abi")
    assert again.cached


@pytest.mark.parametrize(
    "name, kernels, arena",
    [
        ("resnet50", {"gemm": 54, "pool": 1, "reduce": 1, "transpose": 1, "view": 1}, 7225344),
        ("mobilenet_v2", {"depthwise": 17, "gemm": 36, "reduce": 1, "transpose": 1, "view": 1}, 6021120),
        ("tiny-cnn", {"depthwise": 1, "gemm": 9, "pool": 1, "reduce": 1, "transpose": 1, "view": 1}, None),
    ],
)
def test_kernel_mix_matches_reference(name, kernels, arena, monkeypatch):
    """Reference kernel mixes at O3: ResNet-50 gemm 54, pool 1, reduce 1, transpose 1, view 1;
    MobileNetV2 gemm 36, depthwise 17 (benchmarks/results/ablation_cnn.json:759-830,1468-1540);
    tiny-cnn gemm 9, depthwise 1 (tests/test_codegen.py:638-647). With the space-to-depth stem
    the input Transpose folds into the stem's copy, and with ResNet-50's stem launch into that
    launch's image reads; the planned arena is the same every way."""
    from ml_graph_compiler.codegen import hip as hip_codegen

    make = builders.SAMPLES.get(name) or builders.CONFIGS[name]
    monkeypatch.setattr(hip_codegen, "FUSE_PROJECTION_SHORTCUT", False)
    monkeypatch.setattr(hip_codegen, "FUSE_DEPTHWISE_POINTWISE", False)
    monkeypatch.setattr(hip_codegen, "FUSE_STEM_BLOCK", False)
    monkeypatch.setattr(hip_codegen, "FUSE_EXPAND_DEPTHWISE", False)
    monkeypatch.setattr(hip_codegen, "SPACE_TO_DEPTH", False)
    monkeypatch.setattr(hip_codegen, "CONV_STEM", False)
    monkeypatch.setattr(hip_codegen, "FUSE_POOL_FC", False)
    gen = generate_hip(o3(make()))
    assert gen.kernels == kernels
    if arena is not None:
        assert gen.arena_bytes == arena == gen.plan.arena_bytes
    monkeypatch.setattr(hip_codegen, "SPACE_TO_DEPTH", True)
    s2d = generate_hip(o3(make()))
    moved = dict(kernels, folded=1, space_to_depth=1)
    del moved["transpose"]
    assert s2d.kernels == moved
    assert s2d.plan.arena_bytes == gen.plan.arena_bytes
    # ResNet-50's 7 x 7 stem reads the NCHW image in place as one mgc_hip_conv_stem launch
    monkeypatch.setattr(hip_codegen, "CONV_STEM", True)
    stem = generate_hip(o3(make()))
    if name == "resnet50":
        moved = dict(moved, gemm=kernels["gemm"] - 1, gemm_stem=1)
        del moved["space_to_depth"]
    assert stem.kernels == moved
    assert stem.plan.arena_bytes == gen.plan.arena_bytes
    # at batch 1 the global average pooling runs in the launch of the classifier that reads it
    # (all three networks end GlobalAveragePool -> Flatten -> Gemm)
    monkeypatch.setattr(hip_codegen, "FUSE_POOL_FC", True)
    head = generate_hip(o3(make()))
    moved = dict(moved, gemm=moved["gemm"] - 1, folded=moved.get("folded", 0) + 1, pool_fc=1)
    del moved["reduce"]
    assert head.kernels == moved
    assert gen.weights.nbytes % 256 == 0 and len(gen.weights.digest()) == 24
    assert "mgc_forward" in gen.source and "int mgc_run(" in gen.source


def test_stem_launch_at_every_batch():
    """ResNet-50's stem runs as one mgc_hip_conv_stem launch at batch 1 and at batch 32 (no
    space-to-depth copy, the input Transpose read in place)."""
    for batch in (1, 32):
        gen = generate_hip(o3(builders.resnet50(batch=batch)))
        assert gen.kernels.get("gemm_stem") == 1 and "space_to_depth" not in gen.kernels, batch
        assert "transpose" not in gen.kernels, batch


def test_bert_embedding_runs_as_one_launch():
    """BERT-base's token lookup, the position embeddings added to it and the first LayerNorm run
    as one mgc_hip_gather_layer_norm launch at batch 1 and 16 (the (1, 128, 768) position addend
    repeats over the batch); the token ids stay alive until that launch reads them."""
    from ml_graph_compiler.codegen import hip as hip_codegen

    for batch in (1, 16):
        g = o3(builders.bert_base(batch=batch, layers=1))
        fused = hip_codegen.find_gather_layer_norm(g)
        assert len(fused) == 1
        (gather, add, other, add_rows, store_sum), = fused.values()
        assert add_rows == 128 and other.tensor_type.shape == (1, 128, 768) and not store_sum
        gen = generate_hip(g)
        assert gen.kernels.get("gather_layer_norm") == 1 and "gather" not in gen.kernels, gen.kernels
        assert "gl.rows = %dL; gl.cols = 768;" % (128 * batch) in gen.source


def test_gpt2_embedding_runs_as_one_launch_that_stores_the_sum():
    """GPT-2's token lookup plus position embeddings is both the first LayerNorm's input and the
    first residual: the one launch also stores the sum, which the residual reads later."""
    from ml_graph_compiler.codegen import hip as hip_codegen

    g = o3(builders.gpt2(batch=1, layers=1))
    fused = hip_codegen.find_gather_layer_norm(g)
    (gather, add, other, add_rows, store_sum), = fused.values()
    assert store_sum and add_rows == 128
    gen = generate_hip(g)
    assert gen.kernels.get("gather_layer_norm") == 1 and "gather" not in gen.kernels, gen.kernels
    assert "gl.sum = NULL" not in gen.source and "gl.sum = ((float *)" in gen.source


def test_projection_shortcuts_join_their_block_gemm():
    """ResNet-50's four downsample blocks each lose their shortcut GEMM; the shortcut input
    stays alive (its arena block clear of everything placed) until the fused GEMM reads it."""
    from ml_graph_compiler.codegen.hip import find_projection_shortcuts

    g = o3(builders.resnet50())
    pairs = find_projection_shortcuts(g)
    assert len(pairs) == 4
    gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats)
    # 53 convolutions and the classifier: the stem launch, four shortcut GEMMs in their blocks'
    # GEMMs, and at batch 1 the classifier in the pooling launch (pool_fc)
    assert gen.kernels["gemm_shortcut"] == 4 and gen.kernels["gemm"] == 48 and gen.kernels["gemm_stem"] == 1
    assert gen.kernels["pool_fc"] == 1
    assert gen.source.count("g.k1 = ") == 4
    # the shortcut's FLOPs are timed with the GEMM that computes them
    from ml_graph_compiler import ops
    assert sum(gen.node_flops) == sum(ops.flops(n) for n in g.nodes)
    assert all(gen.node_flops[i] == 0 for i, n in enumerate(g.nodes) if id(n) in {id(d) for d in pairs.values()})
    order = {id(n): i for i, n in enumerate(g.nodes)}
    by_value = {id(v): b for b in gen.plan.buffers for v in b.values}
    for c3 in g.nodes:
        ds = pairs.get(id(c3))
        if ds is None:
            continue
        x = by_value[id(ds.input(0))]
        assert x.end >= order[id(c3)]
        for b in gen.plan.buffers:
            if b is x or not (b.start <= order[id(c3)] <= b.end):
                continue
            assert b.offset + b.size <= x.offset or x.offset + x.size <= b.offset
    assert not find_projection_shortcuts(o3(builders.bottleneck()))  # identity shortcuts only


def test_depthwise_pointwise_pairs_join_one_gemm(monkeypatch):
    """MobileNetV2 at batch 32: the six depthwise -> projection pairs whose GEMMs have at least
    DEPTHWISE_FUSE_MIN_ROWS rows (the 112 x 112, 56 x 56 and 28 x 28 outputs) each run as one
    mgc_hip_gemm_dw call; the depthwise input stays alive (its arena block clear of everything
    placed) until that call reads it, and the depthwise FLOPs are counted at the call's node. At
    batch 1 only the two shallow pairs (32 and 96 channels) are fused."""
    from ml_graph_compiler import ops
    from ml_graph_compiler.codegen import hip as emitter
    from ml_graph_compiler.codegen.hip import find_depthwise_pointwise

    monkeypatch.setattr(emitter, "FUSE_INVERTED_RESIDUAL", False)  # whole blocks: the next test
    monkeypatch.setattr(emitter, "FUSE_EXPAND_DEPTHWISE", False)  # expansion + depthwise: below
    g = o3(builders.mobilenet_v2(batch=32))
    pairs = find_depthwise_pointwise(g)
    assert len(pairs) == 6
    assert all(dw.output.tensor_type.shape[1] in (112, 56, 28) for dw in pairs.values())
    assert len(find_depthwise_pointwise(g, min_rows=0)) == 17
    gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats)
    assert gen.kernels["gemm_depthwise"] == 6 and gen.kernels["depthwise"] == 11 and gen.kernels["gemm"] == 36
    assert gen.source.count("mgc_hip_gemm_dw(x, &g, &d);") == 6
    assert sum(gen.node_flops) == sum(ops.flops(n) for n in g.nodes)
    skipped = {id(d) for d in pairs.values()}
    assert all(gen.node_flops[i] == 0 for i, n in enumerate(g.nodes) if id(n) in skipped)
    order = {id(n): i for i, n in enumerate(g.nodes)}
    by_value = {id(v): b for b in gen.plan.buffers for v in b.values}
    for pw in g.nodes:
        dw = pairs.get(id(pw))
        if dw is None:
            continue
        x = by_value[id(dw.input(0))]
        assert x.end >= order[id(pw)]
        for b in gen.plan.buffers:
            if b is x or not (b.start <= order[id(pw)] <= b.end):
                continue
            assert b.offset + b.size <= x.offset or x.offset + x.size <= b.offset
    shallow = find_depthwise_pointwise(o3(builders.mobilenet_v2(batch=1)))  # 112 x 112 = 12544 rows
    assert sorted(dw.input(0).tensor_type.shape[3] for dw in shallow.values()) == [32, 96]


def test_inverted_residual_blocks_run_as_one_launch(monkeypatch):
    """MobileNetV2 at batch 32: the five expanded blocks whose outputs have at least
    MBCONV_MIN_ROWS pixels (56 x 56 and 28 x 28, both strides, 16 / 24 / 32 input channels) each
    run as one mgc_hip_mbconv call, and the stem with the first block (no expansion) as one
    mgc_hip_mbconv_stem call reading the NCHW input in place (the input Transpose, the stem and
    the depthwise convolution emit nothing; no space-to-depth copy). The block input stays
    alive (its arena block clear of everything placed) until the call reads it, and the
    expansion (stem) and depthwise FLOPs are counted at the call's node. At batch 1 only the
    stem block is fused (MBCONV_STEM_MIN_ROWS)."""
    from ml_graph_compiler import ops
    from ml_graph_compiler.codegen import hip as emitter
    from ml_graph_compiler.codegen.hip import find_inverted_residuals

    monkeypatch.setattr(emitter, "FUSE_EXPAND_DEPTHWISE", False)  # the smaller blocks: the next test
    g = o3(builders.mobilenet_v2(batch=32))
    blocks = find_inverted_residuals(g)
    shapes = sorted((ex.input(0).tensor_type.shape[1:], dw.output.tensor_type.shape[1:]) for ex, dw in blocks.values())
    assert shapes == [((28, 28, 32), (28, 28, 192))] * 2 + [((56, 56, 24), (28, 28, 144)), ((56, 56, 24), (56, 56, 144)),
                                                            ((112, 112, 16), (56, 56, 96)), ((224, 224, 3), (112, 112, 32))]
    gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats)
    assert gen.kernels["gemm_mbconv"] == 6 and gen.kernels["mbconv_stem"] == 1 and gen.kernels["depthwise"] == 11
    assert "gemm_depthwise" not in gen.kernels and "space_to_depth" not in gen.kernels and "transpose" not in gen.kernels
    assert gen.source.count("mgc_hip_mbconv(x, &g, &mb);") == 5
    assert gen.source.count("mgc_hip_mbconv_stem(x, &g, &mb, &st);") == 1
    assert "st.sn = 150528L; st.sc = 50176L; st.sh = 224L; st.sw = 1L;" in gen.source  # NCHW [32, 3, 224, 224]
    assert sum(gen.node_flops) == sum(ops.flops(n) for n in g.nodes)
    skipped = {id(n) for pair in blocks.values() for n in pair}
    assert all(gen.node_flops[i] == 0 for i, n in enumerate(g.nodes) if id(n) in skipped)
    order = {id(n): i for i, n in enumerate(g.nodes)}
    by_value = {id(v): b for b in gen.plan.buffers for v in b.values}
    for pw in g.nodes:
        pair = blocks.get(id(pw))
        if pair is None:
            continue
        x = by_value[id(pair[0].input(0))]
        assert x.end >= order[id(pw)]
        for b in gen.plan.buffers:
            if b is x or not (b.start <= order[id(pw)] <= b.end):
                continue
            assert b.offset + b.size <= x.offset or x.offset + x.size <= b.offset
    b1 = find_inverted_residuals(o3(builders.mobilenet_v2(batch=1)))
    assert [ex.input(1).tensor_type.shape[:3] for ex, _ in b1.values()] == [(3, 3, 3)]
    monkeypatch.setattr(emitter, "FUSE_STEM_BLOCK", False)
    assert not find_inverted_residuals(o3(builders.mobilenet_v2(batch=1)))


def test_expansion_and_depthwise_run_as_one_launch():
    """MobileNetV2 at batch 32: the ten expanded blocks on 14 x 14 and 7 x 7 inputs (64, 96 and
    160 input channels, the 14 -> 7 block at stride 2) run their expansion and depthwise
    convolution as one mgc_hip_expand_dw call writing the depthwise output (384-960 workgroups
    of an image and 32 channels each); the projection stays a GEMM. Only the 28 -> 14 block
    (28 x 28 input: too large a window) keeps its depthwise launch, so with the five whole-block
    launches and the stem block one standalone depthwise launch is left of 17. The block input stays alive (its arena block clear of everything placed) until the
    call reads it, the expansion FLOPs are counted at the call's node, and batches 1 and 8 fuse
    the same ten pairs (6-30 and 48-240 workgroups: still ahead of two launches)."""
    from ml_graph_compiler import ops
    from ml_graph_compiler.codegen.hip import expand_dw_supported, find_expand_depthwise

    g = o3(builders.mobilenet_v2(batch=32))
    pairs = find_expand_depthwise(g)
    shapes = sorted((ex.input(0).tensor_type.shape[1:], dw.output.tensor_type.shape[1:]) for dw_id, ex in pairs.items()
                    for dw in g.nodes if id(dw) == dw_id)
    assert shapes == ([((7, 7, 160), (7, 7, 960))] * 3 + [((14, 14, 64), (14, 14, 384))] * 4
                      + [((14, 14, 96), (7, 7, 576))] + [((14, 14, 96), (14, 14, 576))] * 2)
    gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats)
    assert gen.kernels["expand_depthwise"] == 10 and gen.kernels["depthwise"] == 1
    assert gen.kernels["gemm_mbconv"] == 6 and "gemm_depthwise" not in gen.kernels and gen.kernels["gemm"] == 20
    assert gen.source.count("mgc_hip_expand_dw(x, &xd);") == 10
    assert sum(gen.node_flops) == sum(ops.flops(n) for n in g.nodes)
    skipped = {id(ex) for ex in pairs.values()}
    assert all(gen.node_flops[i] == 0 for i, n in enumerate(g.nodes) if id(n) in skipped)
    order = {id(n): i for i, n in enumerate(g.nodes)}
    by_value = {id(v): b for b in gen.plan.buffers for v in b.values}
    for dw in g.nodes:
        ex = pairs.get(id(dw))
        if ex is None:
            continue
        x = by_value[id(ex.input(0))]
        assert x.end >= order[id(dw)]
        for b in gen.plan.buffers:
            if b is x or not (b.start <= order[id(dw)] <= b.end):
                continue
            assert b.offset + b.size <= x.offset or x.offset + x.size <= b.offset
    for batch in (1, 8):
        small = find_expand_depthwise(o3(builders.mobilenet_v2(batch=batch)))
        assert len(small) == 10, batch
    # the kernel's limits: window and row blocks per wave, per input width
    assert expand_dw_supported(14, 14, 96, 576, 2, 7, 7) and expand_dw_supported(16, 14, 64, 32, 2, 8, 7)
    assert not expand_dw_supported(28, 28, 32, 192, 2, 14, 14)
    assert not expand_dw_supported(14, 16, 64, 32, 1, 14, 16)  # window 16 x 18 = 288 pixels
    assert not expand_dw_supported(14, 14, 160, 960, 1, 14, 14)  # 160 channels: at most 64 pixels
    assert not expand_dw_supported(7, 7, 160, 944, 1, 7, 7)  # a partial 32-channel slice


def test_fusions_stay_below_the_fused_kernels_operand_limit(monkeypatch):
    """The fused projection-shortcut and depthwise GEMMs address their operands with 32-bit byte
    offsets and refuse operands of 2 GiB or more at launch, so the emitter must not choose them
    there: ResNet-50 at batch 700 (stage 2's shortcut input [700, 56, 56, 256] is 2.25 GB) and
    MobileNetV2 at batch 450 (the 112 x 112 x 96 depthwise input is 2.17 GB) compile with those
    pairs left to the unfused kernels, and every launch the source counts stays below the limit."""
    from ml_graph_compiler.codegen import hip as emitter

    limit = emitter.FUSED_OPERAND_LIMIT
    nbytes = emitter._tensor_bytes
    monkeypatch.setattr(emitter, "FUSE_INVERTED_RESIDUAL", False)  # (its own limit: the next test)
    for make, find, kind in ((lambda: builders.resnet50(batch=700), emitter.find_projection_shortcuts, "gemm_shortcut"),
                             (lambda: builders.mobilenet_v2(batch=450), emitter.find_depthwise_pointwise, "gemm_depthwise")):
        g = o3(make())
        pairs = find(g)
        with monkeypatch.context() as m:
            m.setattr(emitter, "FUSED_OPERAND_LIMIT", 1 << 62)
            unlimited = find(g)
        dropped = [n for n in g.nodes if id(n) in unlimited and id(n) not in pairs]
        assert len(dropped) == 1, kind
        big = unlimited[id(dropped[0])].input(0)
        assert nbytes(big) >= limit > max(nbytes(p.input(0)) for p in pairs.values())
        gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats)
        assert gen.kernels[kind] == len(pairs) == len(unlimited) - 1


def test_every_sample_and_config_generates_and_builds(hip_cache):
    for name, make in list(builders.SAMPLES.items()) + [("single_gemm", builders.single_gemm), ("bottleneck", builders.bottleneck)]:
        for level in ("O0", "O3"):
            g = make()
            optimize(g, level)
            schedule(g)
            gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats,
                               gemm_ln_workspace=native.gemm_layer_norm_workspace_floats)
            native.build_model_library(gen.source, cache_dir=hip_cache, name="m")
            if name == "tiny-bert" and level == "O3":  # the fused GEMM + LayerNorm call compiles too
                assert gen.kernels.get("gemm_layer_norm", 0) > 0, gen.kernels


def test_split_k_workspace_is_planned():
    g = o3(builders.single_gemm())
    gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats)
    assert native.gemm_workspace_floats(128, 3072, 768, 1) > 0
    assert gen.plan.workspaces and "g.workspace = ((float *)(A + " in gen.source
    assert gen.arena_bytes >= 4 * native.gemm_workspace_floats(128, 3072, 768, 1)


def test_packed_weights_layout():
    b = np.arange(5 * 14, dtype=np.float32).reshape(5, 14)
    packed = pack_b_nk(b)
    assert packed.shape == (14, 5) and packed.flags.c_contiguous
    np.testing.assert_array_equal(packed, b.T)


def test_unsupported_programs_raise():
    g, _ = op_graph("Trilu", [f32(3, 3)])
    with pytest.raises(CodegenError, match="Trilu"):
        generate_hip(g)
    g, _ = op_graph("Pad", [f32(2, 3), np.asarray([1, 1, 1, 1], np.int64)], const={1}, attrs={"mode": "reflect"})
    with pytest.raises(CodegenError, match="reflect"):
        generate_hip(g)
    g, _ = op_graph("Sqrt", [np.ones((2,), np.int64)])
    with pytest.raises(CodegenError, match="Sqrt on int64"):
        generate_hip(g)
    h = Graph()
    x = h.add_input("h", TensorType("float16", (2,)))
    node = h.add_node("Relu", [x])
    node.output.type = TensorType("float16", (2,))
    h.add_output(node.output)
    with pytest.raises(CodegenError, match="float16"):
        generate_hip(h)


def test_hostile_names_cannot_escape_comments(hip_cache):
    g = Graph("g */ int g_injected; /*")
    x = g.add_input("x", TensorType("float32", (2, 3)))
    node = g.add_node("Relu", [x], name="relu */ int injected = 1; /* \n#include <stdlib.h>\n")
    node.output.type = TensorType("float32", (2, 3))
    g.add_output(node.output, "y")
    source = generate_hip(g).source
    assert "*/ int injected" not in source and "*/ int g_injected" not in source
    assert "\n#include <stdlib.h>" not in source
    native.build_model_library(source, cache_dir=hip_cache, name="hostile")


def test_build_errors_are_reported(hip_cache):
    with pytest.raises(CodegenError, match="build failed"):
        native.build_model_library("this is not C++", cache_dir=hip_cache, name="bad")


def test_loading_without_a_gpu_fails_loudly(hip_cache):
    if native.load_kernel_library().mgc_hip_device_count() > 0:
        pytest.skip("a GPU is visible")
    from ml_graph_compiler.codegen import compile_graph

    with pytest.raises(CodegenError, match="no HIP device"):
        compile_graph(o3(builders.mlp()), cache_dir=hip_cache)


def test_other_backends_and_onnx_paths_are_rejected(hip_cache):
    from ml_graph_compiler.codegen import compile_graph, compile_model

    with pytest.raises(CodegenError, match="not part of this build"):
        compile_graph(o3(builders.mlp()), cache_dir=hip_cache, backend="c")
    with pytest.raises(ModelImportError):
        compile_model("model.onnx")


def test_depthwise_detection():
    g = o3(builders.tiny_cnn())
    assert sum(HipEmitter.depthwise(n) for n in g.nodes) == 1


def test_reference_vector_cases_the_backend_rejects():
    """The reference-generated operator cases that neither the reference's C backend nor this
    backend compiles (Trilu; MatMul on int64) fail at generation with a CodegenError naming
    the cause; every other case compiles (tests/test_gpu_reference_vectors.py runs them)."""
    from test_gpu_reference_vectors import UNSUPPORTED
    from test_reference_op_vectors import MANIFEST, decode_attrs, load_case

    with np.load(ROOT / "tests" / "golden" / "reference_ops.npz") as data:
        arrays = {k: data[k] for k in data.files}
    for case in MANIFEST:
        inputs, _ = load_case(case, arrays)
        g, _ = op_graph(case["op"], inputs, const=set(case["const"]), attrs=decode_attrs(case["attrs"]),
                        n_outputs=case["outputs"])
        optimize(g, "O0")
        schedule(g)
        if case["name"] in UNSUPPORTED:
            with pytest.raises(CodegenError, match=UNSUPPORTED[case["name"]]):
                generate_hip(g)
        else:
            generate_hip(g)


def test_gemm_family_flops_are_the_algorithmic_work():
    """The emitter's count of the GEMM-family launches' algorithmic FLOPs (what the profiles'
    TFLOP/s divide): ResNet-50 is 8,178,368,512 per image (the 53 convolutions and the FC, with
    the space-to-depth stem counted as the original 7 x 7 convolution and the projection
    shortcuts at the launches that compute them), less the FC's 2 x 2048 x 1000 per image at the
    batches where the classifier runs in the pooling launch (mgc_hip_pool_fc, not an MFMA kernel);
    BERT-base is everything but the attention products (4 B H S^2 D per layer, which the attention
    kernel computes)."""
    from ml_graph_compiler import ops
    from ml_graph_compiler.codegen import hip as hip_codegen

    gen = generate_hip(o3(builders.resnet50(batch=2)), gemm_workspace=native.gemm_workspace_floats)
    assert gen.kernels.get("pool_fc") == 1
    assert gen.gemm_flops == 2 * (8_178_368_512 - 2 * 2048 * 1000)
    batch = hip_codegen.POOL_FC_MAX_BATCH + 1
    gen = generate_hip(o3(builders.resnet50(batch=batch)), gemm_workspace=native.gemm_workspace_floats)
    assert "pool_fc" not in gen.kernels
    assert gen.gemm_flops == batch * 8_178_368_512
    g = o3(builders.bert_base(batch=1, layers=2))
    gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats,
                       gemm_ln_workspace=native.gemm_layer_norm_workspace_floats)
    contractions = sum(ops.flops(n) for n in g.nodes if n.op in ("FusedGemm", "MatMul", "Gemm"))
    assert gen.gemm_flops == contractions - 2 * 4 * 12 * 128 * 128 * 64
