"""Recognizes scaled dot-product attention in a scheduled graph for the fused hip kernel.

The transformer graphs the reference builds (samples.py:178-245, the BERT config) express
attention as a chain of separate nodes. After O3 (passes/fusion.py) one layer reads:

    qkv = FusedGemm(x, W, b)                       [B, S, 3 * H * D]
    q, k, v = Split(qkv, axis=-1)                  3 x [B, S, H * D]
    tq = Transpose(Reshape(q, [B, S, H, D]), perm=[0, 2, 1, 3])
    tk = Transpose(Reshape(k, [B, S, H, D]), perm=[0, 2, 3, 1])
    tv = Transpose(Reshape(v, [B, S, H, D]), perm=[0, 2, 1, 3])
    t = score ops (MatMul(tq, tk))                 [B, H, S, Skv]
    o = Transpose(MatMul(Softmax(t, axis=-1), tv), perm=[0, 2, 1, 3])  (then Reshape to [B, S, H*D])

The score ops between QK^T and the softmax are, in this order and each optional: a scale
(Mul or Div by a scalar constant), an additive bias (Add of a float tensor that broadcasts
over [B, H, S, Skv], e.g. BERT's padding mask) and a mask (Where(mask, t, fill) or
Where(mask, fill, t) with a scalar constant fill, e.g. GPT's causal mask). They may be separate
nodes or one FusedElementwise program (passes/loopfuse.py). A constant mask that keeps exactly
the keys j <= s is recognized as causal, so the kernel needs no mask tensor and can skip key
blocks past the diagonal.

``find_attention`` returns, for each such chain, the nodes a single mgc_hip_attention call
replaces and the strided views it reads. The memory plan is not touched: the fused call writes
the final Transpose's planned output, and the intermediate values simply never get written.
A chain is taken only where that is safe: every intermediate has no other reader and is not a
graph output, and no other node scheduled between the chain's first and last node writes over
memory the fused call reads. Where the planner reused the (by then
dead) memory of an operand for the output, the match is marked ``staged``: the call writes a
scratch area past the planned arena and a copy moves the result into place.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np

from ..ir import Graph, Node, Value
from ..memory import MemoryPlan

ATT_DMAX = 64   # head dim limit of the kernel (csrc/attention.hip)
# Run the Q/K/V projection GEMM(s) inside the fused call, into scratch (tests turn it off to
# exercise the staged output of a plain match).
ABSORB_QKV = True
SCORE_OPS = ("Mul", "Div", "Add", "Where")


@dataclass
class Operand:
    value: Value      # tensor holding the rows ([B, S, width])
    col: int          # element offset of the head-0 columns within a row
    row_stride: int   # elements between consecutive sequence positions
    batch_stride: int


@dataclass
class ScoreOps:
    """What happens to t = Q K^T before the softmax: t = t * scale (t / scale when
    ``divide``), t += bias, t = keep ? t : fill."""

    scale: float = 1.0
    divide: bool = False
    bias: Value | None = None
    mask: Value | None = None
    mask_keep: bool = True       # keep the score where the mask element is true (else false)
    fill: float = 0.0
    causal: bool = False         # the mask is the constant "key <= query" pattern

    def leaves(self) -> list[Value]:
        return [v for v in (self.bias, self.mask) if v is not None]


@dataclass
class AttentionMatch:
    B: int
    H: int
    S: int
    Skv: int
    D: int
    scale: float
    q: Operand
    k: Operand
    v: Operand
    out: Value                       # the head-merge Transpose output [B, S, H, D]
    emit_at: Node                    # where the fused call goes (that Transpose)
    absorbed: list[Node] = field(default_factory=list)
    staged: bool = False             # output overlaps an operand: write scratch, then copy
    ops: ScoreOps = field(default_factory=ScoreOps)
    # Q, K and V projected by three FusedGemms of one input (Hugging Face exports), or by one
    # FusedGemm whose output only the absorbed Split reads: the fused call runs them as one GEMM
    # with the weights side by side, into a [B*S, 3*H*D] scratch area that the attention kernel
    # then reads like a fused QKV projection.
    qkv_gemms: list[Node] = field(default_factory=list)

    def reads(self) -> list[Value]:
        """Values the fused call reads from memory the plan manages."""
        if self.qkv_gemms:
            return [self.qkv_gemms[0].input(0), *self.ops.leaves()]
        return [self.q.value, self.k.value, self.v.value, *self.ops.leaves()]


def _only_user(value: Value, node: Node, graph: Graph) -> bool:
    return len(value.users) == 1 and value.users[0] is node and value not in graph.outputs


def _perm(node: Node) -> list[int]:
    return [int(p) for p in node.attrs.get("perm", [])]


def _scalar(value: Value) -> float | None:
    if value.data is None or value.data.size != 1:
        return None
    return float(value.data.reshape(-1)[0])


def _head_view(t: Value, perm: list[int], use: Node, graph: Graph) -> tuple[Value, list[Node]] | None:
    """t = Transpose(Reshape(src, [B, S, H, D]), perm) -> (src [B, S, H*D], [reshape, transpose])."""
    tr = t.producer
    if tr is None or tr.op != "Transpose" or _perm(tr) != perm or not _only_user(t, use, graph):
        return None
    r = tr.input(0)
    rs = r.producer
    if rs is None or rs.op != "Reshape" or not _only_user(r, tr, graph):
        return None
    src = rs.input(0)
    if src.type is None or r.type is None or src.type.rank != 3 or r.type.rank != 4:
        return None
    b, s, hd = src.type.shape
    b2, s2, h, d = r.type.shape
    if (b, s) != (b2, s2) or h * d != hd:
        return None
    return src, [rs, tr]


def find_attention(graph: Graph, plan: MemoryPlan) -> list[AttentionMatch]:
    order = {id(n): i for i, n in enumerate(graph.nodes)}
    found: list[AttentionMatch] = []
    for sm in graph.nodes:
        m = _match(sm, graph)
        if m is None:
            continue
        lo = min(order[id(n)] for n in m.absorbed)
        hi = max(order[id(n)] for n in m.absorbed)
        if m.emit_at is not graph.nodes[hi]:
            continue
        reads = m.reads()
        ids = {id(n) for n in m.absorbed}
        if not all(_harmless(graph.nodes[i], i, reads, order, plan)
                   for i in range(lo, hi + 1) if id(graph.nodes[i]) not in ids):
            continue
        # The planner may have put the output where a dead operand was (the QKV projection, a
        # bias); the fused call then writes a scratch area past the planned arena and copies.
        # (A grouped projection's input is consumed by its GEMM before the output is written.)
        attn_reads = m.ops.leaves() if m.qkv_gemms else reads
        m.staged = any(_overlap(plan, v, m.out) for v in attn_reads)
        found.append(m)
    return found


def _harmless(node: Node, at: int, reads: list[Value], order: dict[int, int], plan: MemoryPlan) -> bool:
    """A node the schedule put between the chain's first and last node (say, the computation of
    a bias) still runs before the fused call, so once a value the call reads exists, the node
    must not write over it: the planner may have reused the memory of an operand whose last
    reader was an absorbed node. (Absorbed intermediates have no other readers, so such a node
    cannot read one.)"""
    if id(node) in plan.workspaces:
        return False
    for r in reads:
        born = order.get(id(r.producer), -1) if r.producer is not None else -1
        if at > born and any(_overlap(plan, out, r) for out in node.outputs):
            return False
    return True


def _overlap(plan: MemoryPlan, a: Value, b: Value) -> bool:
    la, lb = plan.location(a), plan.location(b)
    if la.kind != lb.kind or la.kind in ("const",):
        return False
    if la.kind in ("input", "output"):
        return la.index == lb.index
    a0, b0 = la.index, lb.index
    return a0 < b0 + b.tensor_type.nbytes and b0 < a0 + a.tensor_type.nbytes


# -- the score ops between QK^T and the softmax -------------------------------------------------

_Expr = tuple[Any, ...]  # ("S", matmul) | ("leaf", value) | (op, [children])


def _leads_to_matmul(v: Value | None, depth: int = 0) -> bool:
    if v is None or depth > 8:
        return False
    p = v.producer
    if p is None:
        return False
    if p.op == "MatMul":
        return True
    if p.op in SCORE_OPS or p.op == "FusedElementwise":
        return any(_leads_to_matmul(u, depth + 1) for u in p.inputs)
    return False


def _score_expr(v: Value, consumer: Node, graph: Graph, absorbed: list[Node]) -> _Expr | None:
    """Expression tree of a value on the score path (the path from QK^T to the softmax)."""
    p = v.producer
    if p is None or not _only_user(v, consumer, graph):
        return None
    if p.op == "MatMul":
        return ("S", p)
    on_path = [i for i, u in enumerate(p.inputs) if _leads_to_matmul(u)]
    if len(on_path) != 1 or len(p.outputs) != 1:
        return None
    if p.op in SCORE_OPS:
        absorbed.append(p)
        inner = _score_expr(p.inputs[on_path[0]], p, graph, absorbed)
        if inner is None:
            return None
        return (p.op, [inner if i == on_path[0] else ("leaf", u) for i, u in enumerate(p.inputs)])
    if p.op == "FusedElementwise":
        absorbed.append(p)
        inner = _score_expr(p.inputs[on_path[0]], p, graph, absorbed)
        if inner is None:
            return None
        n = len(p.inputs)
        results: list[_Expr] = []
        for op, attrs, args in p.attrs.get("program", []):
            if op not in SCORE_OPS or attrs or any(a < 0 or a >= n + len(results) for a in args):
                return None
            kids = [results[a - n] if a >= n else inner if a == on_path[0] else ("leaf", p.inputs[a]) for a in args]
            results.append((op, kids))
        return results[-1] if results else None
    return None


def _on_path(e: _Expr) -> bool:
    return e[0] != "leaf"


def _broadcasts(v: Value, shape: tuple[int, ...]) -> bool:
    t = v.type
    if t is None or t.rank > len(shape):
        return False
    return all(d in (1, full) for d, full in zip(t.shape, shape[len(shape) - t.rank :]))


def _score_ops(e: _Expr, score_shape: tuple[int, ...]) -> tuple[ScoreOps, Node] | None:
    """Peel Where, then Add, then Mul/Div off the tree (the order the kernel applies them in
    reverse); what remains must be QK^T itself."""
    ops = ScoreOps()
    if e[0] == "Where":
        c, a, b = e[1]
        if c[0] != "leaf" or c[1].type is None or c[1].type.dtype != "bool" or not _broadcasts(c[1], score_shape):
            return None
        if _on_path(a) and not _on_path(b):
            keep, fill, e = True, b[1], a
        elif _on_path(b) and not _on_path(a):
            keep, fill, e = False, a[1], b
        else:
            return None
        f = _scalar(fill)
        if f is None or fill.type is None or fill.type.dtype != "float32":
            return None
        ops.mask, ops.mask_keep, ops.fill = c[1], keep, f
    if e[0] == "Add":
        x, y = e[1]
        path, other = (x, y) if _on_path(x) else (y, x)
        if _on_path(other) or other[1].type is None or other[1].type.dtype != "float32":
            return None
        if not _broadcasts(other[1], score_shape):
            return None
        ops.bias, e = other[1], path
    if e[0] in ("Mul", "Div"):
        x, y = e[1]
        if e[0] == "Div" and not _on_path(x):
            return None
        path, other = (x, y) if _on_path(x) else (y, x)
        if _on_path(other):
            return None
        c = _scalar(other[1])
        if c is None or c == 0.0 or other[1].type is None or other[1].type.dtype != "float32":
            return None
        ops.scale, ops.divide, e = c, e[0] == "Div", path
    if e[0] != "S":
        return None
    if ops.mask is not None and ops.mask.data is not None:
        ops.causal = _is_causal(ops.mask.data, ops.mask_keep, score_shape)
    return ops, e[1]


def _is_causal(mask: np.ndarray, keep_set: bool, score_shape: tuple[int, ...]) -> bool:
    """True when the constant mask keeps exactly the keys j <= s in every (batch, head)."""
    S, Skv = score_shape[-2:]
    keep = np.broadcast_to(np.asarray(mask, bool), score_shape) == keep_set
    return bool(np.array_equal(keep, np.broadcast_to(np.tril(np.ones((S, Skv), bool)), score_shape)))


def _match(sm: Node, graph: Graph) -> AttentionMatch | None:
    if sm.op != "Softmax":
        return None
    x = sm.input(0)
    if x.type is None or x.type.rank != 4 or x.type.dtype != "float32":
        return None
    axis = int(sm.attrs.get("axis", -1))
    if axis not in (-1, 3):
        return None
    absorbed = [sm]
    expr = _score_expr(x, sm, graph, absorbed)
    if expr is None:
        return None
    found = _score_ops(expr, x.type.shape)
    if found is None:
        return None
    ops, qk = found
    absorbed.append(qk)
    p = sm.output
    if len(p.users) != 1 or p in graph.outputs:
        return None
    pv = p.users[0]
    if pv.op != "MatMul" or pv.input(0) is not p:
        return None
    absorbed.append(pv)
    o = pv.output
    if len(o.users) != 1 or o in graph.outputs:
        return None
    tr = o.users[0]
    if tr.op != "Transpose" or _perm(tr) != [0, 2, 1, 3]:
        return None
    absorbed.append(tr)
    tq, tk, tv = qk.input(0), qk.input(1), pv.input(1)
    views = []
    for t, perm, use in ((tq, [0, 2, 1, 3], qk), (tk, [0, 2, 3, 1], qk), (tv, [0, 2, 1, 3], pv)):
        hv = _head_view(t, perm, use, graph)
        if hv is None:
            return None
        views.append(hv[0])
        absorbed += hv[1]
    qs, ks, vs = views
    for v in (qs, ks, vs, tq, tk, tv, o, p, qk.output):
        if v.type is None or v.type.dtype != "float32":
            return None
    B, H, S, D = tq.type.shape
    Skv = tk.type.shape[3]
    if tk.type.shape != (B, H, D, Skv) or tv.type.shape != (B, H, Skv, D) or o.type.shape != (B, H, S, D):
        return None
    if x.type.shape != (B, H, S, Skv) or not (Skv >= 1 and 4 <= D <= ATT_DMAX and D % 4 == 0):
        return None
    HD = H * D
    operands = None
    sp = qs.producer
    if (sp is not None and sp.op == "Split" and len(sp.outputs) == 3 and list(sp.outputs) == [qs, ks, vs]
            and all(_only_user(v, v.users[0] if v.users else sp, graph) for v in (qs, ks, vs))
            and int(sp.attrs.get("axis", -1)) in (-1, 2)):
        src = sp.input(0)
        if src.type is not None and src.type.shape == (B, S, 3 * HD) and S == Skv and src.type.dtype == "float32":
            row = 3 * HD
            operands = [Operand(src, j * HD, row, S * row) for j in range(3)]
            absorbed.append(sp)
    if operands is None:
        if qs.type.shape != (B, S, HD) or ks.type.shape != (B, Skv, HD) or vs.type.shape != (B, Skv, HD):
            return None
        operands = [Operand(qs, 0, HD, S * HD), Operand(ks, 0, HD, Skv * HD), Operand(vs, 0, HD, Skv * HD)]
    if HD % 4:
        return None
    m = AttentionMatch(B=B, H=H, S=S, Skv=Skv, D=D, scale=ops.scale, q=operands[0], k=operands[1],
                       v=operands[2], out=tr.output, emit_at=tr, absorbed=absorbed, ops=ops)
    if not ABSORB_QKV:
        gemms = []
    elif sp is None or sp.op != "Split":
        gemms = _qkv_gemms(m, graph)
    else:
        gemms = _fused_qkv_gemm(sp, m, graph)
    if gemms:
        m.qkv_gemms = gemms
        m.absorbed += gemms
    return m


def _fused_qkv_gemm(sp: Node, m: AttentionMatch, graph: Graph) -> list[Node]:
    """The FusedGemm whose [B, S, 3HD] output only the absorbed Split reads (a model with Q, K
    and V weights already side by side): it runs as part of the fused call, into scratch, so the
    attention output never shares memory with its operands and needs no staging copy."""
    src = sp.input(0)
    p = src.producer
    if p is None or src in graph.outputs or len(src.users) != 1 or _gemm_form(p) is None:
        return []
    a = p.input(0)
    if a.type is None or a.type.dtype != "float32" or a.type.size != m.B * m.S * a.type.shape[-1]:
        return []
    return [p]


def _gemm_form(node: Node) -> tuple[Any, ...] | None:
    if node.op != "FusedGemm" or node.optional_input(3) is not None or node.input(1).data is None:
        return None
    bias = node.optional_input(2)
    if bias is not None and (bias.data is None or bias.data.size != node.output.tensor_type.shape[-1]):
        return None
    return (id(node.input(0)), int(node.attrs.get("trans_b", 0)), str(node.attrs.get("activation", "none")),
            float(node.attrs.get("clip_min", 0.0)), float(node.attrs.get("clip_max", 6.0)), bias is None,
            node.input(1).tensor_type.shape)


def _qkv_gemms(m: AttentionMatch, graph: Graph) -> list[Node]:
    """The three FusedGemms of one input that produce Q, K and V, when their outputs feed only
    the head-split Reshapes this chain absorbs."""
    nodes = []
    for op in (m.q, m.k, m.v):
        v = op.value
        p = v.producer
        if p is None or v in graph.outputs or len(v.users) != 1 or v.users[0].op != "Reshape":
            return []
        nodes.append(p)
    if len({id(n) for n in nodes}) != 3 or m.S != m.Skv:
        return []
    forms = [_gemm_form(n) for n in nodes]
    if forms[0] is None or any(f != forms[0] for f in forms):
        return []
    a = nodes[0].input(0)
    if a.type is None or a.type.dtype != "float32" or a.type.size != m.B * m.S * a.type.shape[-1]:
        return []
    return nodes
