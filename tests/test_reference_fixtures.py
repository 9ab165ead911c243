"""The compiler pipeline against the reference implementation's own outputs.

tests/golden/reference_plans.json was written by tests/golden/make_reference_fixtures.py, which
ran the reference's passes, scheduler and planner (src/ml_graph_compiler/passes, schedule.py,
memory.py) on the same builder graphs. What it pins exactly, and what tolerance-based tests
cannot: the O3 operator mix and node order, the memory-aware schedule statistics, and every
planned location (kind and byte offset) at alignment 256 (hip) and 64 (C backend).
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from ml_graph_compiler import builders
from ml_graph_compiler.memory import plan_memory
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule

FIXTURE = json.loads((Path(__file__).parent / "golden" / "reference_plans.json").read_text())

CASES = {
    "mlp": builders.mlp,
    "tiny-cnn": builders.tiny_cnn,
    "tiny-gpt": builders.tiny_gpt,
    "tiny-bert": builders.tiny_bert,
    "single_gemm": builders.single_gemm,
    "bottleneck_b1": lambda: builders.bottleneck(1),
    "bottleneck_b32": lambda: builders.bottleneck(32),
    "resnet50_b1": lambda: builders.resnet50(1),
    "mobilenet_v2_b1": lambda: builders.mobilenet_v2(1),
    "bert_base_b1": lambda: builders.bert_base(1),
    "tiny_transformer_separate_qkv": lambda: builders.transformer(separate_qkv=True),
    "tiny_transformer_erf": lambda: builders.transformer(gelu="erf", causal=False),
    "bert_2l_b2_separate_qkv": lambda: builders.bert_base(2, layers=2, separate_qkv=True),
    "gpt2_2l_b1": lambda: builders.gpt2(1, layers=2),
    "mobilenet_v2_b2": lambda: builders.mobilenet_v2(2),
    "resnet50_b2": lambda: builders.resnet50(2),
    "bottleneck_b3": lambda: builders.bottleneck(3),
}


def _describe(graph, alignment):
    plan = plan_memory(graph, alignment=alignment)
    locs = []
    for node in graph.nodes:
        for v in node.outputs:
            loc = plan.location(v)
            locs.append([node.op, loc.kind, int(loc.index)])
    return {
        "arena_bytes": plan.arena_bytes,
        "lower_bound": plan.lower_bound,
        "naive_bytes": plan.naive_bytes,
        "buffers": len(plan.buffers),
        "inplace": plan.inplace,
        "aliases": plan.aliases,
        "copies": [j for _, j in plan.copies],
        "locations": locs,
    }


@pytest.mark.parametrize("name", sorted(CASES))
def test_pipeline_schedule_and_plan_match_reference(name):
    expected = FIXTURE[name]
    graph = CASES[name]()
    assert len(graph.nodes) == expected["nodes_o0"]
    optimize(graph, "O3")
    report = schedule(graph)
    assert graph.op_counts() == expected["ops_o3"]
    assert [n.op for n in graph.nodes] == expected["order"]
    got = {"peak_before": report.peak_before, "peak_after": report.peak_after, "levels": report.levels,
           "max_width": report.max_width, "critical_flops": report.critical_flops, "total_flops": report.total_flops}
    assert got == expected["schedule"]
    for alignment in (256, 64):
        assert _describe(graph, alignment) == expected[f"plan{alignment}"], alignment


def test_resnet50_arena_matches_published_figure():
    """README.md:246 of the reference: ResNet-50 arena 7,225,344 bytes (greedy by size)."""
    assert FIXTURE["resnet50_b1"]["plan64"]["arena_bytes"] == 7225344
    assert FIXTURE["mobilenet_v2_b1"]["plan64"]["arena_bytes"] == 6021120
