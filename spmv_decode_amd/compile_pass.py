"""torch.compile pass: sibling `nmsparse::gemv` calls become one launch, with
the RMSNorm in front of them and the residual add after them folded in.

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
  problems each (one grouped launch), whose outputs replace the calls';
* then an RMSNorm in front of a launch (rmsnorm(x) * weight over the last
  axis, in the forms model code writes it: _rms_norm) folds into it: the
  launch reads x and applies the norm as it gathers (a lone gemv becomes a
  one-problem gemv_grouped), and the norm's nodes go when nothing else uses
  them (fold_input_norms);
* and a residual add of a gemv's output (add(r, gemv(...)), same shape, fp16,
  the output used for nothing else) becomes one `nmsparse::gemv_residual`
  launch that adds r in fp32 before its one rounding (fold_residuals).

It runs as inductor's post-grad pre-pass (torch._inductor.config.
post_grad_custom_pre_pass), installed when the package is imported unless
NM_COMPILE_GROUPING=0; a pass the user installed before stays, and runs first.
Graphs without `nmsparse::gemv` nodes are left untouched. The rewrite changes
which kernel computes a projection, not what it computes: each output is the
same fp32-accumulated sum rounded once (the grouped plan may split the
columns differently, so the last bit of a sum can differ; the SiLU product,
the normalised input and the residual sum are formed in fp32 and rounded
once instead of twice, as the decoder's fused layer does).
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
                    args = (x, g.args[1], g.args[2], u.args[1], u.args[2], g.args[3], g.args[4], g.args[5], g.args[6],
                            None, 0.0)
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
                    [n.args[4] for n in chunk], chunk[0].args[5], chunk[0].args[6], None, 0.0)
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


def _rms_norm(node):
    """(x, weight, eps) when `node` is an RMSNorm of the 16-bit x over its last
    axis times weight ([K], x's dtype), as model code writes it and inductor
    decomposes it: n = x32 * rsqrt(mean(x32^2, -1, keepdim) + eps), x32 = x
    in fp32, then either convert(n * weight) to x's dtype (weight applied in
    fp32) or convert(n) * weight (weight applied after the rounding, as the
    Hugging Face and gpt-fast norms do); else None."""
    aten, prims = torch.ops.aten, torch.ops.prims

    def convert_of(n, dtype):
        if _is(n, prims.convert_element_type.default) and n.args[1] == dtype:
            return n.args[0]
        return None

    def mul_pair(n):
        if _is(n, aten.mul.Tensor) and len(n.args) == 2 and not n.kwargs:
            return n.args
        return None

    def normalized(n):  # n = x32 * rsqrt(mean(x32 ** 2) + eps) -> (x, eps)
        ab = mul_pair(n)
        if ab is None:
            return None
        for x32, r in (ab, ab[::-1]):
            if not (_is(r, aten.rsqrt.default) and isinstance(x32, torch.fx.Node)):
                continue
            add = r.args[0]
            if not (any(_is(add, t) for t in (aten.add.Scalar, aten.add_.Scalar, aten.add.Tensor))
                    and len(add.args) == 2 and isinstance(add.args[1], (int, float)) and not add.kwargs):
                continue
            mean, eps = add.args
            if not (_is(mean, aten.mean.dim) and len(mean.args) >= 3 and mean.args[2] is True):
                continue
            sq, dims = mean.args[0], list(mean.args[1])
            square = ((_is(sq, aten.pow.Tensor_Scalar) and sq.args[0] is x32 and sq.args[1] == 2)
                      or (mul_pair(sq) is not None and sq.args[0] is x32 and sq.args[1] is x32))
            x = convert_of(x32, torch.float32)
            xv = _fake(x)
            if not square or not isinstance(xv, torch.Tensor) or xv.dtype not in (torch.float16, torch.bfloat16):
                continue
            if dims not in ([-1], [xv.dim() - 1]):
                continue
            return x, float(eps)
        return None

    def weight_ok(wn, x):
        wv, xv = _fake(wn), _fake(x)
        return (isinstance(wn, torch.fx.Node) and isinstance(wv, torch.Tensor) and wv.dtype == xv.dtype
                and tuple(wv.shape) == (xv.shape[-1],))

    # weight applied in fp32, then one rounding
    inner = None
    if _is(node, prims.convert_element_type.default) and node.args[1] in (torch.float16, torch.bfloat16):
        inner = node.args[0]
    if inner is not None:
        ab = mul_pair(inner)
        if ab is not None:
            for n, wn in (ab, ab[::-1]):
                got = normalized(n) if isinstance(n, torch.fx.Node) else None
                if got is not None and weight_ok(wn, got[0]) and _fake(node).dtype == _fake(got[0]).dtype:
                    return got[0], wn, got[1]
    # the rounding first, then the weight (in x's dtype)
    ab = mul_pair(node)
    if ab is not None:
        for c, wn in (ab, ab[::-1]):
            if not _is(c, prims.convert_element_type.default):
                continue
            got = normalized(c.args[0])
            if got is not None and c.args[1] == _fake(got[0]).dtype and weight_ok(wn, got[0]):
                return got[0], wn, got[1]
    return None


def _erase_if_unused(graph, nodes):
    """Erase the nodes of `nodes` (in order) that nothing uses any more, after
    their own users that nothing uses and that have no side effects (a view
    left over, say)."""
    for n in nodes:
        if not (isinstance(n, torch.fx.Node) and n.op == "call_function") or n.is_impure():
            continue
        for u in list(n.users):
            if u.op == "call_function" and not u.users and not u.is_impure():
                graph.erase_node(u)
        if not n.users:
            graph.erase_node(n)


def _chain(node, stop):
    """`node` and the nodes it reads, back to (not including) `stop`, latest first."""
    seen, order, todo = set(), [], [node]
    while todo:
        n = todo.pop()
        if n in seen or n is stop or not isinstance(n, torch.fx.Node) or n.op != "call_function":
            continue
        seen.add(n)
        order.append(n)
        todo.extend(a for a in n.all_input_nodes)
    pos = {n: i for i, n in enumerate(node.graph.nodes)}
    return sorted(order, key=pos.get, reverse=True)


def fold_input_norms(graph: torch.fx.Graph) -> int:
    """Fold an RMSNorm in front of gemv launches into them: a `gemv`,
    `gemv_grouped` or `gemv_silu_mul` node whose input is rmsnorm(x) * weight
    (_rms_norm) reads x instead, with the norm's weight and eps (a single gemv
    becomes a one-problem gemv_grouped). The norm's nodes are removed when
    nothing else uses them. Returns the number of launches rewritten."""
    gemv, grouped, silu_mul = _ops()
    done = 0
    for n in list(graph.nodes):
        if not (_is(n, gemv) or _is(n, grouped) or _is(n, silu_mul)):
            continue
        if (_is(n, grouped) or _is(n, silu_mul)) and n.args[-2] is not None:
            continue  # already folded
        normed = n.args[0]
        got = _rms_norm(normed) if isinstance(normed, torch.fx.Node) else None
        if got is None or _fake(got[0]).dtype != torch.float16:
            continue
        x, weight, eps = got
        if _is(n, gemv):
            if len(n.args) != 7 or n.kwargs:
                continue
            _, md, mi, w, h, bw, vw = n.args
            args = (x, [md], [mi], w, [h], bw, vw, weight, eps)
            with graph.inserting_before(n):
                node = graph.call_function(grouped, args)
                _set_meta(node, grouped, args)
                item = graph.call_function(operator.getitem, (node, 0))
                if "val" in node.meta:
                    item.meta["val"] = node.meta["val"][0]
            n.replace_all_uses_with(item)
            graph.erase_node(n)
        else:
            args = (x, *n.args[1:-2], weight, eps)
            n.args = args
            if "val" in n.meta:
                _set_meta(n, n.target, args)
        _erase_if_unused(graph, _chain(normed, x))
        done += 1
    if done:
        graph.lint()
    return done


def fold_residuals(graph: torch.fx.Graph) -> int:
    """Fold a residual add into the gemv in front of it: add(r, gemv(...)) (in
    either order, same shape, fp16, the gemv used by nothing else) becomes
    one `gemv_residual` node. Returns the number of adds folded."""
    aten = torch.ops.aten
    gemv = torch.ops.nmsparse.gemv.default
    target = torch.ops.nmsparse.gemv_residual.default
    done = 0
    for n in list(graph.nodes):
        if not (_is(n, aten.add.Tensor) and len(n.args) == 2 and not n.kwargs):
            continue
        for r, y in (n.args, n.args[::-1]):
            if not (_is(y, gemv) and len(y.args) == 7 and not y.kwargs and len(y.users) == 1
                    and isinstance(r, torch.fx.Node)):
                continue
            rv, yv, nv = _fake(r), _fake(y), _fake(n)
            if not all(isinstance(v, torch.Tensor) for v in (rv, yv, nv)):
                continue
            if not (rv.dtype == yv.dtype == nv.dtype == torch.float16 and rv.shape == yv.shape == nv.shape):
                continue
            args = (*y.args, r)
            with graph.inserting_before(n):
                node = graph.call_function(target, args)
                _set_meta(node, target, args)
            n.replace_all_uses_with(node)
            graph.erase_node(n)
            graph.erase_node(y)
            done += 1
            break
    if done:
        graph.lint()
    return done


class SiblingGemvPass(CustomGraphPass):
    """group_sibling_gemvs, then fold_input_norms and fold_residuals, as an
    inductor custom graph pass (its uuid keys inductor's graph cache to this
    file's contents)."""

    def __init__(self, before=None):
        self.before = before  # a pass installed earlier, run first

    def __call__(self, graph: torch.fx.Graph) -> None:
        if self.before is not None:
            self.before(graph)
        group_sibling_gemvs(graph)
        fold_input_norms(graph)
        fold_residuals(graph)

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


__all__ = ["group_sibling_gemvs", "fold_input_norms", "fold_residuals", "SiblingGemvPass", "install", "uninstall"]
