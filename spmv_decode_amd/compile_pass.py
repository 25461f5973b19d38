"""torch.compile pass: sibling `nmsparse::gemv` calls become one launch.

Model code written for dense Linears calls each projection on its own, so a
swapped model issues one `nmsparse::gemv` per Linear (the reference's decode
step does exactly that: src/spmv/nmsparse_linear.py:62-68). In eager mode the
sibling ties of nmsparse_linear.SiblingLaunch group them at run time; under
torch.compile that host bookkeeping cannot run, so this pass does the grouping
on the compiled graph instead, where data flow is explicit:

* `gemv` nodes that read the same input node with the same w and N:M (q/k/v
  of a Hugging Face attention block, w1/w3 of a gpt-fast feed-forward block)
  are siblings;
* a sibling pair whose outputs meet as silu(gate) * up (the SiLU-gated MLP;
  after inductor's decompositions: convert to fp32, sigmoid, multiply, convert
  back, multiply by up) becomes one `nmsparse::gemv_silu_mul` node: the
  gate/up pair kernel with the SiLU and the product in its epilogue;
* the remaining siblings become `nmsparse::gemv_grouped` nodes of 2-4
  problems each (one grouped launch), whose outputs replace the calls'.

It runs as inductor's post-grad pre-pass (torch._inductor.config.
post_grad_custom_pre_pass), installed when the package is imported unless
NM_COMPILE_GROUPING=0; a pass the user installed before stays, and runs first.
Graphs without `nmsparse::gemv` nodes are left untouched. The rewrite changes
which kernel computes a projection, not what it computes: each output is the
same fp32-accumulated sum rounded once (the grouped plan may split the
columns differently, so the last bit of a sum can differ; the SiLU product
is formed in fp32 and rounded once instead of twice).
No reference counterpart.
"""
from __future__ import annotations

import operator
import os

import torch
from torch._inductor.custom_graph_pass import CustomGraphPass, get_hash_for_files

_ENABLED = os.environ.get("NM_COMPILE_GROUPING", "1")
if _ENABLED not in ("0", "1"):
    raise ValueError(f"Unknown NM_COMPILE_GROUPING={_ENABLED!r}; use 0 or 1")

MAX_GROUP = 4  # problems per grouped launch (include/nmsparse_hip.h: nm_gemv_launch_desc.prob)


def _ops():
    ops = torch.ops.nmsparse
    return ops.gemv.default, ops.gemv_grouped.default, ops.gemv_silu_mul.default


def _is(node, target) -> bool:
    return isinstance(node, torch.fx.Node) and node.op == "call_function" and node.target is target


def _only_user(node):
    users = list(node.users)
    return users[0] if len(users) == 1 else None


def _silu_mul_pair(gate, up):
    """The node computing silu(gate) * up from the two gemv outputs, and the
    nodes between them, when the outputs are used only for that (None
    otherwise). Matches silu as one aten.silu node or as inductor decomposes
    it: convert to fp32, x * sigmoid(x), convert back."""
    aten, prims = torch.ops.aten, torch.ops.prims
    g1 = _only_user(gate)
    if g1 is None:
        return None
    inner = []
    if _is(g1, aten.silu.default):
        act = g1
        inner = [g1]
    elif _is(g1, prims.convert_element_type.default) and g1.args[1] == torch.float32:
        users = set(g1.users)
        sig = next((u for u in users if _is(u, aten.sigmoid.default)), None)
        mul = next((u for u in users if _is(u, aten.mul.Tensor)), None)
        if sig is None or mul is None or users != {sig, mul} or _only_user(sig) is not mul:
            return None
        if set(mul.args) != {g1, sig}:
            return None
        back = _only_user(mul)
        if back is None or not _is(back, prims.convert_element_type.default) or back.args[1] != torch.float16:
            return None
        act = back
        inner = [g1, sig, mul, back]
    else:
        return None
    prod = _only_user(act)
    if prod is None or not _is(prod, aten.mul.Tensor) or set(prod.args) != {act, up} or _only_user(up) is not prod:
        return None
    return prod, inner


def _fake(node):
    return node.meta.get("val") if isinstance(node, torch.fx.Node) else node


def _set_meta(new, target, args):
    """node.meta['val'] of a new node: its op run on the arguments' fake values."""
    vals = torch.fx.node.map_arg(args, _fake)
    fake_mode = next((v.fake_mode for v in torch.utils._pytree.tree_leaves(vals)
                      if isinstance(v, torch._subclasses.FakeTensor)), None)
    if fake_mode is None:
        return
    with fake_mode:
        new.meta["val"] = target(*vals)


def group_sibling_gemvs(graph: torch.fx.Graph) -> int:
    """Rewrite sibling gemv nodes of `graph` in place (see the module
    docstring); returns the number of gemv nodes replaced."""
    gemv, grouped, silu_mul = _ops()
    order = {n: i for i, n in enumerate(graph.nodes)}
    families = {}
    for n in graph.nodes:
        if _is(n, gemv) and len(n.args) == 7 and not n.kwargs:
            x, md, mi, w, h, bw, vw = n.args
            families.setdefault((x, w, bw, vw), []).append(n)
    replaced = 0
    for members in families.values():
        if len(members) < 2:
            continue
        members.sort(key=order.get)
        first = members[0]
        # every operand must exist before the first sibling: parameters and constants are placeholders or
        # get_attr nodes (which read nothing and can move); anything computed later keeps its call apart
        ok = []
        for n in members:
            movable = True
            for a in n.args[1:3]:
                if isinstance(a, torch.fx.Node) and order[a] > order[first] and a.op != "get_attr":
                    movable = False
            if movable:
                for a in n.args[1:3]:
                    if isinstance(a, torch.fx.Node) and a.op == "get_attr" and order[a] > order[first]:
                        first.prepend(a)
                ok.append(n)
        order = {n: i for i, n in enumerate(graph.nodes)}
        x = first.args[0]
        x_val = _fake(x)
        pending = list(ok)
        # SiLU-gated pairs first (fp16 inputs: the pair kernel rounds the product to fp16 once)
        if isinstance(x_val, torch.Tensor) and x_val.dtype == torch.float16:
            for g in list(pending):
                for u in list(pending):
                    if g is u or g not in pending or u not in pending or g.args[4] != u.args[4]:
                        continue
                    m = _silu_mul_pair(g, u)
                    if m is None:
                        continue
                    prod, inner = m
                    args = (x, g.args[1], g.args[2], u.args[1], u.args[2], g.args[3], g.args[4], g.args[5], g.args[6])
                    with graph.inserting_before(first):
                        node = graph.call_function(silu_mul, args)
                    _set_meta(node, silu_mul, args)
                    prod.replace_all_uses_with(node)
                    for dead in [prod] + inner[::-1] + [g, u]:
                        graph.erase_node(dead)
                    if g is first or u is first:
                        first = node
                    pending.remove(g)
                    pending.remove(u)
                    replaced += 2
        for i in range(0, len(pending), MAX_GROUP):
            chunk = pending[i:i + MAX_GROUP]
            if len(chunk) < 2:
                continue
            args = (x, [n.args[1] for n in chunk], [n.args[2] for n in chunk], chunk[0].args[3],
                    [n.args[4] for n in chunk], chunk[0].args[5], chunk[0].args[6])
            anchor = min(chunk, key=lambda n: order.get(n, -1)) if first not in chunk else first
            with graph.inserting_before(anchor):
                node = graph.call_function(grouped, args)
                _set_meta(node, grouped, args)
                outs = []
                for j in range(len(chunk)):
                    item = graph.call_function(operator.getitem, (node, j))
                    if "val" in node.meta:
                        item.meta["val"] = node.meta["val"][j]
                    outs.append(item)
            for n, item in zip(chunk, outs):
                n.replace_all_uses_with(item)
                graph.erase_node(n)
            replaced += len(chunk)
    if replaced:
        graph.lint()
    return replaced


class SiblingGemvPass(CustomGraphPass):
    """group_sibling_gemvs as an inductor custom graph pass (its uuid keys
    inductor's graph cache to this file's contents)."""

    def __init__(self, before=None):
        self.before = before  # a pass installed earlier, run first

    def __call__(self, graph: torch.fx.Graph) -> None:
        if self.before is not None:
            self.before(graph)
        group_sibling_gemvs(graph)

    def uuid(self):
        before = self.before.uuid() if isinstance(self.before, CustomGraphPass) else repr(self.before)
        return (get_hash_for_files((os.path.abspath(__file__),)), before)


def install() -> bool:
    """Install the pass as inductor's post-grad pre-pass (once; an existing
    pass is kept and runs first). Returns whether the pass is installed."""
    import torch._inductor.config as inductor_config

    current = inductor_config.post_grad_custom_pre_pass
    if isinstance(current, SiblingGemvPass):
        return True
    if _ENABLED == "0":
        return False
    inductor_config.post_grad_custom_pre_pass = SiblingGemvPass(before=current)
    return True


def uninstall() -> None:
    """Remove the pass (restoring any pass it wrapped)."""
    import torch._inductor.config as inductor_config

    current = inductor_config.post_grad_custom_pre_pass
    if isinstance(current, SiblingGemvPass):
        inductor_config.post_grad_custom_pre_pass = current.before


__all__ = ["group_sibling_gemvs", "SiblingGemvPass", "install", "uninstall"]
