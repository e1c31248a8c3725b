"""Model converter that moves a torchtitan-style model's LoRA linears onto libwsl.

Follows the reference's converter protocol (torchtitan/protocols/model_converter.py:15-33):
constructed with ``(job_config, parallel_dims)``, ``convert(model)`` rewrites the model in
place, ``post_optimizer_hook(model)`` runs after each optimizer step; converters are
registered by name (:36-50) and applied by the trainer (torchtitan/train.py:160-161).

The reference's attention holds each LoRA projection as a base ``nn.Linear`` and a
``LoRAModule`` offset and composes them in its forward (model.py:239-330, 376-398):

    default        xq = broadcast_add(self.wq_base(x), self.wq_offset(x), g)        (base as wide as q)
    head_sharing   the same call, wq_base holding g templates of width D' < q's width
    qkv_sharing    val = getattr(self, str(group))(x); q_base = k_base = v_base = val;
                   xq = broadcast_add(q_base, self.wq_offset(x), g), likewise k and v

    two_step       head_offset = self.head_offset(x)                                  (as wide as q)
                   wq_offset = broadcast_add(self.wq_only_offset(x), head_offset).contiguous()
                   (one head wide, repeated over the heads), likewise k and v; then as above

``WslLoRAConverter.convert`` folds each composition into one launch of the shared-base
fused op (``wsl::lora_linear_bcast``: x . W^T broadcast over the head templates plus the
offset's s (x . A^T) . B^T, never materialising the expanded base or the delta):

- a ``<p>_base`` / ``<p>_offset`` pair (default and head sharing) becomes a ``FusedBase`` and
  a folded offset;
- a shared q/k/v base module becomes a ``FusedSharedBase`` and the group's offsets folded
  offsets;
- under ``two_step`` each projection's offset is the pair (head_offset, w<p>_only_offset): by
  linearity it is one LoRA of rank r_h + r_p with A = [A_h; A_p] and B = [B_h | B_p repeated
  over the heads] (row c of the second block is row c mod D of B_p), so the pair folds into
  the projection's fused launch as one more rank block, and the whole q/k/v set stays one
  launch per base.

The fused modules and folded offsets return zero-stride placeholders that record their
input. The converter swaps the ``broadcast_add`` that the attention's module calls for a
wrapper: given a fused base's placeholder and a folded offset's, it runs the one launch
(with the ``g`` of the call) and returns the projection (its column block for a shared base;
the other projections of the group reuse the same launch); any other call keeps the
original semantics, and a fused base used alone is computed as the plain base. So the
parent's forward is unchanged and pays no extra pass over its outputs. Offsets of the
``two_step`` variant whose bases cannot all be fused, and unpaired LoRA modules, become wsl
``LoRAModule``s (the delta in one launch). Every Parameter object is kept, so optimizer state and state-dict keys
(``<p>_base.weight``, ``<p>_offset.w_a.weight``, ``<p>_offset.w_b.weight``) do not change.
"""
from __future__ import annotations

import sys
from typing import Dict, List, Optional, Union

import torch
import torch.nn as nn

from . import ops
from .lora import LoRAModule

_PENDING = "_wsl_pending"  # on a fused base's placeholder: its _Pending record
_FOLDED = "_wsl_folded"    # on a folded offset's placeholder: its block in the fused output
_TWO_STEP = "_wsl_two_step"  # on a two_step offset's placeholder: ("head", None) or ("only", (block, width))


class _Pending:
    """A fused base's call: its input and the fused outputs computed from it, by g."""

    def __init__(self, x: torch.Tensor, owner: nn.Module):
        self.x = x
        self.owner = owner
        self.out: Dict[int, torch.Tensor] = {}


_ZEROS: Dict[torch.device, torch.Tensor] = {}


def _placeholder(x: torch.Tensor, width: int, attr: str, value) -> torch.Tensor:
    """A zero-stride view of one cached zero per device (no device work), tagged."""
    z = _ZEROS.get(x.device)
    if z is None:
        z = _ZEROS[x.device] = torch.zeros((), dtype=torch.bfloat16, device=x.device)
    t = z.expand(*x.shape[:-1], width)
    setattr(t, attr, value)
    return t


_EMPTY: Dict[torch.device, torch.Tensor] = {}


def _contiguous_placeholder(like: torch.Tensor, width: int, attr: str, value) -> torch.Tensor:
    """A contiguous, never-written view of [..., width] bf16 (a cached buffer per device, no
    device work), tagged. The reference calls .contiguous() on a two_step offset, which keeps
    a contiguous tensor (and its tag) as it is."""
    n = like.numel() // max(like.shape[-1], 1) * width
    buf = _EMPTY.get(like.device)
    if buf is None or buf.numel() < n:
        buf = _EMPTY[like.device] = torch.empty(max(n, 1), dtype=torch.bfloat16, device=like.device)
    t = buf[:n].view(*like.shape[:-1], width)
    setattr(t, attr, value)
    return t


def folding_broadcast_add(original):
    """``broadcast_add`` for converted modules. Given a fused base's placeholder and a folded
    offset's, the fused launch of the base's input runs once per ``g`` and the offset's
    column block of it is returned; a fused base's placeholder with any other delta is first
    computed as the plain base x . W^T; every other call is ``original(base, delta, dim=dim,
    g=g)``."""
    def broadcast_add(base, delta, *, dim=-1, g=1):
        ts_base, ts_delta = getattr(base, _TWO_STEP, None), getattr(delta, _TWO_STEP, None)
        if ts_base is not None and ts_delta is not None and ts_base[0] == "only" and ts_delta[0] == "head" \
                and int(g) == 1 and (dim == -1 or dim == base.dim() - 1):
            # broadcast_add(w<p>_only_offset(x), head_offset(x)): the pair is one folded offset
            return _contiguous_placeholder(delta, delta.shape[-1], _FOLDED, ts_base[1])
        if ts_base is not None or ts_delta is not None:
            raise RuntimeError("a folded two_step offset's placeholder met an unexpected broadcast_add")
        pend = getattr(base, _PENDING, None)
        slot = getattr(delta, _FOLDED, None)
        if pend is not None and slot is not None and (dim == -1 or dim == base.dim() - 1):
            out = pend.out.get(int(g))
            if out is None:
                out = pend.owner.fused(pend.x, int(g))
                pend.out[int(g)] = out
            block, width = slot
            return out if out.shape[-1] == width else out.narrow(-1, block * width, width)
        if pend is not None:
            base = pend.owner.plain(pend.x)
        if slot is not None:
            raise RuntimeError("a folded LoRA offset's placeholder met a base that is not its fused base")
        return original(base, delta, dim=dim, g=g)

    broadcast_add._wsl_original = original
    return broadcast_add


class FusedBase(nn.Module):
    """The base half of a fused pair: ``weight`` is the original base Parameter; the LoRA
    factors are read from the paired offset module (held outside the module tree so its
    parameters keep their one state-dict key). Its forward is a placeholder; the projection
    is computed where the module's broadcast_add meets it with the folded offset's."""

    def __init__(self, base: nn.Linear, lora: LoRAModule):
        super().__init__()
        self.weight = base.weight
        self.in_features = base.in_features
        self.out_features = base.out_features
        object.__setattr__(self, "_loras", [lora])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _placeholder(x, self.out_features, _PENDING, _Pending(x, self))

    def plain(self, x: torch.Tensor) -> torch.Tensor:
        return ops.lora_linear(x, self.weight, None, None, 0.0)

    def _build(self):
        ls = self._loras
        if len(ls) == 1:
            return _factors(ls[0])
        fs = [_factors(m) for m in ls]
        return torch.cat([a for a, _ in fs], 0), torch.cat([b for _, b in fs], 0)

    def _stacked(self):
        """[A_0; A_1; ...] and [B_0; B_1; ...] of the offsets. With autograd on they are
        stacked on every call (the stack is differentiable); without, once per parameter
        version."""
        ls = self._loras
        if len(ls) == 1 and not isinstance(ls[0], _TwoStepPair):
            return ls[0].w_a.weight, ls[0].w_b.weight
        if torch.is_grad_enabled():
            return self._build()
        key = tuple((p.data_ptr(), p._version) for m in ls for p in _params(m))
        cache = getattr(self, "_stack_cache", None)
        if cache is None or cache[0] != key:
            cache = (key, *self._build())
            object.__setattr__(self, "_stack_cache", cache)
        return cache[1], cache[2]

    def fused(self, x: torch.Tensor, g: int) -> torch.Tensor:
        """broadcast_add(x . W^T, each offset's delta, g), the offsets side by side."""
        ls = self._loras
        lora = ls[0]
        a, b = self._stacked()
        if len(ls) == 1 and lora.out_dim == self.out_features:
            return ops.lora_linear(x, self.weight, a, b, lora.scale)
        return ops.lora_linear_bcast_op(x, self.weight, None, a, b, float(lora.scale), g, len(ls))

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, fused LoRA "
                f"rank={self._loras[0].rank}, projections={len(self._loras)}")


class _TwoStepPair:
    """The two_step offset of one projection (the reference's model.py:275-300,367-375):
    broadcast_add(w<p>_only_offset(x), head_offset(x)) = s (x . A^T) . B^T with A = [A_h; A_p]
    [r_h + r_p, K] and B = [B_h | B_p repeated over the heads] [N, r_h + r_p] (B_p has D rows;
    output column c takes row c mod D). Not a module: its LoRA modules stay where they are."""

    def __init__(self, head: LoRAModule, only: LoRAModule):
        self.head, self.only = head, only
        self.rank = head.rank + only.rank
        self.scale = head.scale
        self.out_dim = head.out_dim

    def factors(self):
        hb, ob = self.head.w_b.weight, self.only.w_b.weight
        b = torch.cat([hb, ob.repeat(self.out_dim // self.only.out_dim, 1)], 1)
        return torch.cat([self.head.w_a.weight, self.only.w_a.weight], 0), b


def _factors(m):
    """(A [r, K], B [N, r]) of a folded offset."""
    return m.factors() if isinstance(m, _TwoStepPair) else (m.w_a.weight, m.w_b.weight)


def _params(m):
    if isinstance(m, _TwoStepPair):
        return (m.head.w_a.weight, m.head.w_b.weight, m.only.w_a.weight, m.only.w_b.weight)
    return (m.w_a.weight, m.w_b.weight)


class FusedSharedBase(FusedBase):
    """A base shared by several projections (the reference's qkv_sharing): one launch gives
    every projection of the group, side by side, each broadcast_add(base, its offset, g)."""

    def __init__(self, base: nn.Linear, loras: List[LoRAModule]):
        super().__init__(base, loras[0])
        object.__setattr__(self, "_loras", list(loras))


class _FoldedLoRA(LoRAModule):
    """A wsl LoRAModule whose delta is computed inside its fused base's launch: its forward is
    a placeholder for the converted module's ``broadcast_add`` (see the module docstring)."""

    _block = 0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _placeholder(x, self.out_dim, _FOLDED, (self._block, self.out_dim))


class _TwoStepHead(LoRAModule):
    """head_offset of a folded two_step attention: a placeholder for broadcast_add."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _placeholder(x, self.out_dim, _TWO_STEP, ("head", None))


class _TwoStepOnly(LoRAModule):
    """w<p>_only_offset of a folded two_step attention: a placeholder for broadcast_add that
    names the pair's block in its fused base's output (block, width)."""

    _slot = (0, 0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _placeholder(x, self.out_dim, _TWO_STEP, ("only", self._slot))


def _is_lora(m: nn.Module) -> bool:
    """The reference's LoRAModule shape (model.py:148-192): bias-free w_a, w_b, rank, alpha."""
    return (isinstance(getattr(m, "w_a", None), nn.Linear) and isinstance(getattr(m, "w_b", None), nn.Linear)
            and m.w_a.bias is None and m.w_b.bias is None and hasattr(m, "rank") and hasattr(m, "alpha"))


def _as_wsl(m: nn.Module, cls=LoRAModule) -> LoRAModule:
    scale = m.scale if isinstance(m, LoRAModule) else m.alpha / m.rank
    return cls(m.w_a.in_features, m.w_b.out_features, rank=m.rank, w_a_override=m.w_a,
               w_b_override=m.w_b, scale=scale)


def _folded(m: nn.Module, block: int) -> _FoldedLoRA:
    f = _as_wsl(m, _FoldedLoRA)
    f._block = block
    return f


def _is_base(m) -> bool:
    return isinstance(m, nn.Linear) and type(m) is nn.Linear and m.bias is None


class WslLoRAConverter:
    """``model.converters = ["wsl_lora"]``: fused LoRA linears (see the module docstring)."""

    def __init__(self, job_config=None, parallel_dims=None):
        self.fused: List[str] = []       # offsets folded into a fused base
        self.converted: List[str] = []   # other LoRA modules moved to wsl LoRAModule
        self.shared: List[str] = []      # shared q/k/v bases folded with their offsets
        self._patched_modules: List[str] = []

    def _patch(self, parent: nn.Module) -> bool:
        """Swap the broadcast_add the parent's module calls for the folding one. False when
        the module has none (then nothing is folded: the placeholders would be added)."""
        mod = sys.modules.get(type(parent).__module__)
        fn = getattr(mod, "broadcast_add", None) if mod is not None else None
        if fn is None:
            return False
        if getattr(fn, "_wsl_original", None) is None:
            mod.broadcast_add = folding_broadcast_add(fn)
            self._patched_modules.append(mod.__name__)
        return True

    def _fold_two_step(self, pname: str, parent: nn.Module) -> None:
        """The reference's two_step attention (model.py:275-300,367-375): every projection's
        offset is the pair (head_offset, w<p>_only_offset), folded into its base's launch as
        one LoRA of rank r_h + r_p. Taken only when every base can be fused (plain linears:
        one per projection, or the qkv_sharing groups covering q, k and v), the ranks and
        scales agree and the widths broadcast; otherwise the offsets are converted alone."""
        if not getattr(parent, "two_step", False):
            return
        head = getattr(parent, "head_offset", None)
        onlys = {p: getattr(parent, f"w{p}_only_offset", None) for p in "qkv"}
        if not (head is not None and _is_lora(head) and all(o is not None and _is_lora(o) for o in onlys.values())):
            return
        if isinstance(head, _TwoStepHead):
            return
        scale = lambda m: m.scale if isinstance(m, LoRAModule) else m.alpha / m.rank
        mods = [head, *onlys.values()]
        if len({scale(m) for m in mods}) != 1 or len({m.rank for m in onlys.values()}) != 1:
            return
        K = head.w_a.in_features
        D = onlys["q"].w_b.out_features
        if any(o.w_b.out_features != D or o.w_a.in_features != K for o in onlys.values()):
            return
        width = head.w_b.out_features
        if width % D != 0:
            return
        groups = getattr(parent, "qkv_sharing", None)
        if groups:
            if sorted(p for grp in groups for p in grp) != ["k", "q", "v"]:
                return
            plan = [(str(grp), list(grp)) for grp in groups]
        else:
            plan = [(f"w{p}_base", [p]) for p in "qkv"]
        for attr, letters in plan:
            base = getattr(parent, attr, None)
            if not (_is_base(base) and base.in_features == K and width % base.out_features == 0
                    and len(letters) <= ops._native.WSL_MAX_GROUPS):
                return
        if not self._patch(parent):
            return
        h = _as_wsl(head, _TwoStepHead)
        parent.head_offset = h
        path = lambda n: f"{pname}.{n}" if pname else n
        for attr, letters in plan:
            pairs = []
            for j, p in enumerate(letters):
                o = _as_wsl(onlys[p], _TwoStepOnly)
                o._slot = (j, width)
                setattr(parent, f"w{p}_only_offset", o)
                pairs.append(_TwoStepPair(h, o))
                self.fused.append(path(f"w{p}_only_offset"))
            base = getattr(parent, attr)
            setattr(parent, attr, FusedSharedBase(base, pairs) if len(letters) > 1 else FusedBase(base, pairs[0]))
            if len(letters) > 1:
                self.shared.append(path(attr))
        self.fused.append(path("head_offset"))

    def _fold_shared(self, pname: str, parent: nn.Module) -> None:
        groups = getattr(parent, "qkv_sharing", None)
        if not groups or getattr(parent, "two_step", False):
            return
        for grp in groups:
            base = getattr(parent, str(grp), None)
            offs = [getattr(parent, f"w{letter}_offset", None) for letter in grp]
            if not _is_base(base) or not all(o is not None and _is_lora(o) for o in offs):
                continue
            widths = {o.w_b.out_features for o in offs}
            ranks = {o.rank for o in offs}
            scales = {(o.scale if isinstance(o, LoRAModule) else o.alpha / o.rank) for o in offs}
            if len(widths) != 1 or len(ranks) != 1 or len(scales) != 1 or len(offs) > ops._native.WSL_MAX_GROUPS:
                continue
            if widths.pop() % base.out_features != 0 or base.in_features != offs[0].w_a.in_features:
                continue
            if not self._patch(parent):
                continue
            folded = []
            for j, letter in enumerate(grp):
                f = _folded(offs[j], j)
                setattr(parent, f"w{letter}_offset", f)
                folded.append(f)
                self.fused.append(f"{pname}.w{letter}_offset" if pname else f"w{letter}_offset")
            setattr(parent, str(grp), FusedSharedBase(base, folded))
            self.shared.append(f"{pname}.{grp}" if pname else str(grp))

    def convert(self, model: nn.Module) -> None:
        for pname, parent in list(model.named_modules()):
            self._fold_two_step(pname, parent)
            self._fold_shared(pname, parent)
            for name, child in list(parent.named_children()):
                path = f"{pname}.{name}" if pname else name
                if not name.endswith("_offset") or not _is_lora(child) or isinstance(child, _FoldedLoRA):
                    continue
                base = getattr(parent, name[: -len("_offset")] + "_base", None)
                if (_is_base(base) and base.in_features == child.w_a.in_features
                        and child.w_b.out_features % base.out_features == 0 and self._patch(parent)):
                    lora = _folded(child, 0)
                    setattr(parent, name, lora)
                    setattr(parent, name[: -len("_offset")] + "_base", FusedBase(base, lora))
                    self.fused.append(path)
            for name, child in list(parent.named_children()):
                if _is_lora(child) and type(child) not in (LoRAModule, _FoldedLoRA, _TwoStepHead, _TwoStepOnly):
                    setattr(parent, name, _as_wsl(child))
                    self.converted.append(f"{pname}.{name}" if pname else name)

    def post_optimizer_hook(self, model: Union[nn.Module, List[nn.Module]]) -> None:
        return None


_registry: Dict[str, type] = {}


def register_model_converter(converter_cls: type, name: str) -> None:
    """As torchtitan/protocols/model_converter.py:41-50: one class per name."""
    if name in _registry:
        raise ValueError(f"A model converter {name!r} is already registered.")
    _registry[name] = converter_cls


def build_model_converters(names: List[str], job_config=None, parallel_dims=None) -> list:
    return [_registry[n](job_config, parallel_dims) for n in names]


register_model_converter(WslLoRAConverter, "wsl_lora")
