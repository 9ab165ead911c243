"""Recognizes scaled dot-product attention in a scheduled graph for the fused hip kernel.

The transformer graphs the reference builds (samples.py:178-245, the BERT config) express
attention as a chain of separate nodes. After O3 (passes/fusion.py) one layer reads:

    qkv = FusedGemm(x, W, b)                       [B, S, 3 * H * D]
    q, k, v = Split(qkv, axis=-1)                  3 x [B, S, H * D]
    tq = Transpose(Reshape(q, [B, S, H, D]), perm=[0, 2, 1, 3])
    tk = Transpose(Reshape(k, [B, S, H, D]), perm=[0, 2, 3, 1])
    tv = Transpose(Reshape(v, [B, S, H, D]), perm=[0, 2, 1, 3])
    p = Softmax(Mul(MatMul(tq, tk), scale), axis=-1)
    o = Transpose(MatMul(p, tv), perm=[0, 2, 1, 3])  [B, S, H, D]  (then Reshape to [B, S, H*D])

``find_attention`` returns, for each such chain, the nodes a single mgc_hip_attention call
replaces and the strided views it reads. The memory plan is not touched: the fused call writes
the final Transpose's planned output, and the intermediate values simply never get written.
A chain is taken only where that is safe: every intermediate has no other reader and is not a
graph output, and the chain's nodes are contiguous in the schedule, so nothing else writes the
arena between the QKV projection and the fused call. Where the planner reused the (by then
dead) operand memory for the output, the match is marked ``staged``: the call writes a
scratch area past the planned arena and a copy moves the result into place.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from ..ir import Graph, Node, Value
from ..memory import MemoryPlan

ATT_SMAX = 256  # key count limit of the kernel (csrc/attention.hip)
ATT_DMAX = 64   # head dim limit


@dataclass
class Operand:
    value: Value      # tensor holding the rows ([B, S, width])
    col: int          # element offset of the head-0 columns within a row
    row_stride: int   # elements between consecutive sequence positions
    batch_stride: int


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
        ids = {id(n) for n in m.absorbed}
        if any(id(n) not in ids for n in graph.nodes[lo : hi + 1]):
            continue
        if m.emit_at is not graph.nodes[hi]:
            continue
        # The planner may have put the output where the (by then dead) QKV projection was; the
        # fused call then writes a scratch area past the planned arena and copies from there.
        m.staged = any(_overlap(plan, op.value, m.out) for op in (m.q, m.k, m.v))
        found.append(m)
    return found


def _overlap(plan: MemoryPlan, a: Value, b: Value) -> bool:
    la, lb = plan.location(a), plan.location(b)
    if la.kind != lb.kind or la.kind in ("const",):
        return False
    if la.kind in ("input", "output"):
        return la.index == lb.index
    a0, b0 = la.index, lb.index
    return a0 < b0 + b.tensor_type.nbytes and b0 < a0 + a.tensor_type.nbytes


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
    scale = 1.0
    prod = x.producer
    if prod is not None and prod.op in ("Mul", "Div"):
        if not _only_user(x, sm, graph):
            return None
        a, b = prod.input(0), prod.input(1)
        c = _scalar(b)
        s_in = a
        if c is None and prod.op == "Mul":
            c, s_in = _scalar(a), b
        if c is None or c == 0.0:
            return None
        scale = c if prod.op == "Mul" else 1.0 / c
        absorbed.append(prod)
        x_user, x = prod, s_in
    else:
        x_user = sm
    qk = x.producer
    if qk is None or qk.op != "MatMul" or not _only_user(x, x_user, graph):
        return None
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
    for v in (qs, ks, vs, tq, tk, tv, o, x, p):
        if v.type is None or v.type.dtype != "float32":
            return None
    B, H, S, D = tq.type.shape
    Skv = tk.type.shape[3]
    if tk.type.shape != (B, H, D, Skv) or tv.type.shape != (B, H, Skv, D) or o.type.shape != (B, H, S, D):
        return None
    if not (1 <= Skv <= ATT_SMAX and 4 <= D <= ATT_DMAX and D % 4 == 0):
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
    return AttentionMatch(B=B, H=H, S=S, Skv=Skv, D=D, scale=scale, q=operands[0], k=operands[1],
                          v=operands[2], out=tr.output, emit_at=tr, absorbed=absorbed)
