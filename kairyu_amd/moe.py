"""Qwen3-style sparse MoE block with 128x128 block-scaled FP8 experts.

Mirrors the reference's routing and expert mixing
(kairyu/models/moe.py:27-119,255-332: ``_ExpertMlp``, ``_mix_experts``,
``route_experts``' Qwen3 branch, ``Qwen3MoeSparseBlock``) and its packed
expert storage (kairyu/models/grouped_moe.py:46-330: ``GroupedExpertPack``),
with every expert projection a :class:`BlockFp8Linear` (e4m3 weights, fp32
``weight_scale_inv`` per 128x128 block, dynamic 1x128 activation blocks).

On a gfx950 device the whole expert path is one C call
(``kq_moe_block_fp8_experts``): device-side stable sort of the routed rows by
expert, per-token activation quantization, grouped GEMM gate_up with a fused
SwiGLU + 1x128 quantization epilogue, grouped GEMM down, and the fp32
slot-order combine (moe_parallel.py:255-283).  Routing alone is
``kq_moe_route_topk``; the block's forward routes inside the same call
(``kq_moe_routed_block_fp8_experts``), where the routing, the sort's expert
histograms and the token quantization share one launch.  Nothing
synchronizes with the host, so a block can be captured in a HIP graph.  On the CPU the reference's own loop semantics run
(``forward_reference`` of each projection, ``index_add_`` combine).
"""

from __future__ import annotations

import torch
from torch import nn

from kairyu_amd import _native
from kairyu_amd.quant import block_fp8
from kairyu_amd.quant.linear import (
    BlockFp8Linear,
    ExpertScope,
    LinearRole,
    ModelScope,
    make_linear,
)

__all__ = [
    "BlockFp8ExpertMlp",
    "GroupedBlockFp8Experts",
    "Qwen3BlockFp8MoeBlock",
    "mix_experts",
    "route_experts",
    "route_logits",
]


# ------------------------------------------------------------------ routing
def route_logits(
    logits: torch.Tensor, top_k: int, norm_topk_prob: bool = True
) -> tuple[torch.Tensor, torch.Tensor]:
    """Qwen3 routing of ``logits [T, E]`` -> (int64 ``[T, k]``, fp32 ``[T, k]``).

    Stable descending sort (ties -> smaller expert id); weights are the fp32
    softmax of the selected logits (``norm_topk_prob``) or the fp32 softmax of
    all logits gathered at the selection (moe.py:255-273).
    """

    indices, weights = _route(logits, top_k, norm_topk_prob)
    return indices.long(), weights


def _route(logits: torch.Tensor, top_k: int, norm_topk_prob: bool):
    if logits.ndim != 2:
        raise ValueError("router logits must be [tokens, experts]")
    if not logits.is_cuda:
        indices = torch.argsort(logits, dim=-1, descending=True, stable=True)[:, :top_k]
        if norm_topk_prob:
            weights = torch.softmax(logits.gather(1, indices).to(torch.float32), dim=-1)
        else:
            weights = torch.softmax(logits, dim=-1, dtype=torch.float32).gather(1, indices)
        return indices, weights
    logits = logits.contiguous()
    tokens, experts = logits.shape
    indices = torch.empty((tokens, top_k), device=logits.device, dtype=torch.int32)
    weights = torch.empty((tokens, top_k), device=logits.device, dtype=torch.float32)
    _native.call(
        "kq_moe_route_topk", logits.data_ptr(), _native.dtype_code(logits.dtype), tokens, experts,
        top_k, int(bool(norm_topk_prob)), indices.data_ptr(), weights.data_ptr(),
        _native.stream_handle(logits.device),
    )
    return indices, weights


def route_experts(block: nn.Module, hidden: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``route_experts`` (moe.py:255-273) for a block with ``gate``, ``top_k``
    and ``norm_topk_prob``."""

    return route_logits(block.gate(hidden), block.top_k, block.norm_topk_prob)


# ------------------------------------------------------------------ experts
class BlockFp8ExpertMlp(nn.Module):
    """One SwiGLU expert at the checkpoint's (Hugging Face) names:
    ``down(silu(gate(x)) * up(x))`` (``_ExpertMlp``, moe.py:27-83).

    With a ``linear_factory`` the three projections are built through
    :func:`make_linear` with the reference's roles (``MLP_GATE`` / ``MLP_UP``
    column-parallel, ``MLP_DOWN`` row-parallel) and expert identity, so the
    checkpoint's quantization (block FP8 here) and the device kernel binding
    come from the factory; without one they are :class:`BlockFp8Linear`."""

    _kairyu_grouped_swiglu = True

    def __init__(
        self,
        hidden_size: int,
        intermediate_size: int,
        linear_factory=None,
        *,
        prefix: str = "expert",
        layer_index: int | None = None,
        expert_index: int | None = None,
        expert_scope: ExpertScope = ExpertScope.NONE,
        model_scope: ModelScope = ModelScope.TARGET,
    ) -> None:
        super().__init__()
        if linear_factory is None:
            self.gate_proj = BlockFp8Linear(hidden_size, intermediate_size, False)
            self.up_proj = BlockFp8Linear(hidden_size, intermediate_size, False)
            self.down_proj = BlockFp8Linear(intermediate_size, hidden_size, False)
            return
        common = {"layer_index": layer_index, "expert_index": expert_index,
                  "expert_scope": expert_scope, "model_scope": model_scope}
        self.gate_proj = make_linear(linear_factory, hidden_size, intermediate_size, False,
                                     qualified_name=f"{prefix}.gate_proj", role=LinearRole.MLP_GATE,
                                     shard_dim=0, **common)
        self.up_proj = make_linear(linear_factory, hidden_size, intermediate_size, False,
                                   qualified_name=f"{prefix}.up_proj", role=LinearRole.MLP_UP,
                                   shard_dim=0, **common)
        self.down_proj = make_linear(linear_factory, intermediate_size, hidden_size, False,
                                     qualified_name=f"{prefix}.down_proj", role=LinearRole.MLP_DOWN,
                                     shard_dim=1, **common)

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.down_proj(nn.functional.silu(self.gate_proj(hidden)) * self.up_proj(hidden))


class GroupedBlockFp8Experts:
    """Contiguous e4m3 ``gate_up [E, 2I, H]`` / ``down [E, H, I]`` weights and
    their block scales behind the experts' canonical buffers.

    Like the reference's ``GroupedExpertPack`` (grouped_moe.py:143-172) the
    per-expert ``weight`` / ``weight_scale_inv`` buffers become views into the
    packed storage, so checkpoint names do not change and no second copy of
    the weights exists.  Gate rows precede up rows (grouped_moe.py:159-160).
    """

    __slots__ = ("_experts", "w13", "s13", "w2", "s2", "hidden", "inter")

    def __init__(self, experts, w13, s13, w2, s2) -> None:
        self._experts = tuple(experts)
        self.w13, self.s13, self.w2, self.s2 = w13, s13, w2, s2
        self.hidden = w13.shape[2]
        self.inter = w2.shape[2]

    @classmethod
    def from_tensors(cls, w13, s13, w2, s2) -> GroupedBlockFp8Experts:
        """A pack over already-stacked tensors (no expert modules)."""

        experts, inter2, hidden = w13.shape
        inter = inter2 // 2
        if tuple(w2.shape) != (experts, hidden, inter):
            raise ValueError(f"down weights {tuple(w2.shape)} != {(experts, hidden, inter)}")
        if tuple(s13.shape) != (experts, -(-inter2 // 128), -(-hidden // 128)):
            raise ValueError("gate_up block scales do not match the weights")
        if tuple(s2.shape) != (experts, -(-hidden // 128), -(-inter // 128)):
            raise ValueError("down block scales do not match the weights")
        return cls((), w13, s13, w2, s2)

    @classmethod
    def create(cls, experts) -> GroupedBlockFp8Experts | None:
        """Pack homogeneous bias-free block-FP8 SwiGLU experts; None otherwise."""

        experts = tuple(experts)
        if not experts:
            return None
        projections = []
        for expert in experts:
            if type(expert).__dict__.get("_kairyu_grouped_swiglu") is not True:
                return None
            triple = tuple(getattr(expert, name, None) for name in ("gate_proj", "up_proj", "down_proj"))
            if any(not isinstance(m, BlockFp8Linear) or m.bias is not None for m in triple):
                return None
            projections.append(triple)
        gate, up, down = projections[0]
        hidden, inter = gate.in_features, gate.out_features
        if hidden % 128 or inter % 128:
            return None
        device = gate.weight.device
        if device.type == "meta":
            return None
        for g, u, d in projections:
            if (g.in_features, g.out_features, u.in_features, u.out_features,
                    d.in_features, d.out_features) != (hidden, inter, hidden, inter, inter, hidden):
                return None
            if any(m.weight.device != device for m in (g, u, d)):
                return None
        count = len(projections)
        ib, hb = inter // 128, hidden // 128
        with torch.no_grad():
            w13 = torch.empty((count, 2 * inter, hidden), dtype=torch.float8_e4m3fn, device=device)
            s13 = torch.empty((count, 2 * ib, hb), dtype=torch.float32, device=device)
            w2 = torch.empty((count, hidden, inter), dtype=torch.float8_e4m3fn, device=device)
            s2 = torch.empty((count, hb, ib), dtype=torch.float32, device=device)
            for i, (g, u, d) in enumerate(projections):
                w13[i, :inter].copy_(g.weight)
                w13[i, inter:].copy_(u.weight)
                s13[i, :ib].copy_(g.weight_scale_inv)
                s13[i, ib:].copy_(u.weight_scale_inv)
                w2[i].copy_(d.weight)
                s2[i].copy_(d.weight_scale_inv)
        for i, (g, u, d) in enumerate(projections):
            g._buffers["weight"], g._buffers["weight_scale_inv"] = w13[i, :inter], s13[i, :ib]
            u._buffers["weight"], u._buffers["weight_scale_inv"] = w13[i, inter:], s13[i, ib:]
            d._buffers["weight"], d._buffers["weight_scale_inv"] = w2[i], s2[i]
        return cls(experts, w13, s13, w2, s2)

    def is_current(self) -> bool:
        """Whether every expert's buffers still view the packed storage."""

        if not self._experts:
            return True
        storages = {t.untyped_storage().data_ptr() for t in (self.w13, self.s13, self.w2, self.s2)}
        for expert in self._experts:
            for name in ("gate_proj", "up_proj", "down_proj"):
                module = getattr(expert, name, None)
                if not isinstance(module, BlockFp8Linear):
                    return False
                for buf in (module.weight, module.weight_scale_inv):
                    if buf.untyped_storage().data_ptr() not in storages:
                        return False
        return True

    def supports(self, hidden: torch.Tensor) -> bool:
        return (
            hidden.is_cuda
            and hidden.dtype in (torch.float16, torch.bfloat16)
            and hidden.shape[-1] == self.hidden
            and self.w13.device == hidden.device
        )

    def forward(self, hidden: torch.Tensor, topk_indices: torch.Tensor,
                topk_weights: torch.Tensor) -> torch.Tensor:
        """Routed experts + fp32 slot-order combine; ``hidden [T, H]``,
        ``topk_indices [T, k]`` (int32 or int64), ``topk_weights [T, k]``."""

        if not self.supports(hidden):
            raise RuntimeError("block-FP8 grouped experts need fp16/bf16 device rows of the packed width")
        if topk_indices.shape != topk_weights.shape or topk_indices.shape[0] != hidden.shape[0]:
            raise ValueError("one routing row per token is required")
        hidden = hidden.contiguous()
        tokens, top_k = topk_indices.shape
        experts = self.w13.shape[0]
        indices = topk_indices.to(torch.int32).contiguous()
        weights = topk_weights.to(torch.float32).contiguous()
        out = torch.empty_like(hidden)
        if tokens == 0:
            return out
        need = int(_native.library().kq_moe_workspace_size(tokens, self.hidden, self.inter,
                                                            experts, top_k))
        ws = _native.workspace(hidden.device, need)
        _native.call(
            "kq_moe_block_fp8_experts", hidden.data_ptr(), _native.dtype_code(hidden.dtype),
            tokens, self.hidden, self.inter, experts, top_k, indices.data_ptr(), weights.data_ptr(),
            self.w13.data_ptr(), self.s13.data_ptr(), self.w2.data_ptr(), self.s2.data_ptr(),
            out.data_ptr(), ws.data_ptr(), ws.numel(), _native.stream_handle(hidden.device),
        )
        return out

    def forward_logits(self, hidden: torch.Tensor, logits: torch.Tensor, top_k: int,
                       norm_topk_prob: bool = True
                       ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Routing from ``logits [T, E]`` and the routed experts in one library
        call (``kq_moe_routed_block_fp8_experts``): the same outputs, bit for
        bit, as :func:`route_logits` followed by :meth:`forward`.  Returns
        ``(out, topk_indices int32 [T, k], topk_weights fp32 [T, k])``."""

        if not self.supports(hidden):
            raise RuntimeError("block-FP8 grouped experts need fp16/bf16 device rows of the packed width")
        if logits.ndim != 2 or logits.shape[0] != hidden.shape[0]:
            raise ValueError("router logits must be [tokens, experts] with one row per token")
        experts = self.w13.shape[0]
        if logits.shape[1] != experts:
            raise ValueError(f"router logits have {logits.shape[1]} experts, the pack {experts}")
        if logits.device != hidden.device:
            raise ValueError("router logits must be on the hidden states' device")
        hidden = hidden.contiguous()
        logits = logits.contiguous()
        tokens = hidden.shape[0]
        indices = torch.empty((tokens, top_k), device=hidden.device, dtype=torch.int32)
        weights = torch.empty((tokens, top_k), device=hidden.device, dtype=torch.float32)
        out = torch.empty_like(hidden)
        if tokens == 0:
            return out, indices, weights
        need = int(_native.library().kq_moe_workspace_size(tokens, self.hidden, self.inter,
                                                            experts, top_k))
        ws = _native.workspace(hidden.device, need)
        _native.call(
            "kq_moe_routed_block_fp8_experts", logits.data_ptr(), _native.dtype_code(logits.dtype),
            int(bool(norm_topk_prob)), hidden.data_ptr(), _native.dtype_code(hidden.dtype), tokens,
            self.hidden, self.inter, experts, top_k, self.w13.data_ptr(), self.s13.data_ptr(),
            self.w2.data_ptr(), self.s2.data_ptr(), indices.data_ptr(), weights.data_ptr(),
            out.data_ptr(), ws.data_ptr(), ws.numel(), _native.stream_handle(hidden.device),
        )
        return out, indices, weights


# ------------------------------------------------------------------- mixing
def mix_experts(hidden, experts, topk_indices, topk_weights, grouped=None) -> torch.Tensor:
    """``_mix_experts`` (moe.py:86-119): the grouped device path combines in
    fp32 slot order; the reference's loop path (CPU) accumulates per expert
    with ``index_add_`` in fp32; one final cast either way."""

    if grouped is not None and grouped.supports(hidden):
        return grouped.forward(hidden, topk_indices, topk_weights)
    combine_dtype = torch.promote_types(hidden.dtype, topk_weights.dtype)
    out = torch.zeros_like(hidden, dtype=combine_dtype)
    for expert_id in topk_indices.unique():
        token_mask, slot = (topk_indices == expert_id).nonzero(as_tuple=True)
        expert_out = experts[int(expert_id)](hidden[token_mask]).to(combine_dtype)
        weights = topk_weights[token_mask, slot].to(combine_dtype)
        out.index_add_(0, token_mask, expert_out * weights[:, None])
    return out.to(hidden.dtype)


def _refresh_grouped(module: nn.Module, _incompatible_keys=None) -> None:
    current = getattr(module, "_grouped_experts", None)
    if current is not None and current.is_current():
        return
    object.__setattr__(module, "_grouped_experts", GroupedBlockFp8Experts.create(module.experts))


class Qwen3BlockFp8MoeBlock(nn.Module):
    """Qwen3 sparse MoE block (moe.py:276-332) with block-FP8 routed experts:
    ``gate`` (router linear), ``experts.{i}.{gate,up,down}_proj``.

    With a ``linear_factory`` the router (``MOE_ROUTER``: dense by the default
    selection policy) and every routed expert projection (``ROUTED`` scope,
    global expert index) are built through it, as the reference's block does."""

    def __init__(self, hidden_size: int, intermediate_size: int, num_experts: int, top_k: int,
                 norm_topk_prob: bool = True, linear_factory=None, *, prefix: str = "mlp",
                 layer_index: int = 0, model_scope: ModelScope = ModelScope.TARGET) -> None:
        super().__init__()
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        if linear_factory is None:
            self.gate = nn.Linear(hidden_size, num_experts, bias=False)
        else:
            self.gate = make_linear(linear_factory, hidden_size, num_experts, False,
                                    qualified_name=f"{prefix}.gate", model_scope=model_scope,
                                    role=LinearRole.MOE_ROUTER, layer_index=layer_index)
        self.experts = nn.ModuleList(
            BlockFp8ExpertMlp(
                hidden_size, intermediate_size, linear_factory,
                prefix=f"{prefix}.experts.{index}", layer_index=layer_index,
                expert_index=index if linear_factory is not None else None,
                expert_scope=ExpertScope.ROUTED if linear_factory is not None else ExpertScope.NONE,
                model_scope=model_scope,
            )
            for index in range(num_experts)
        )
        _refresh_grouped(self)
        self.register_load_state_dict_post_hook(_refresh_grouped)

    def _apply(self, fn, recurse: bool = True):
        result = super()._apply(fn, recurse=recurse)
        _refresh_grouped(self)
        return result

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        shape = hidden.shape
        flat = hidden.reshape(-1, shape[-1])
        grouped = getattr(self, "_grouped_experts", None)
        if flat.is_cuda and grouped is not None and grouped.supports(flat):
            out, _, _ = grouped.forward_logits(flat, self.gate(flat), self.top_k, self.norm_topk_prob)
            return out.reshape(shape)
        indices, weights = route_experts(self, flat)
        return mix_experts(flat, self.experts, indices, weights).reshape(shape)


def quantize_experts(block: Qwen3BlockFp8MoeBlock, gate_up: torch.Tensor, down: torch.Tensor) -> None:
    """Fill a block's experts from float weights ``gate_up [E, 2I, H]`` (gate
    rows first) and ``down [E, H, I]`` by 128x128 block quantization."""

    inter = down.shape[2]
    with torch.no_grad():
        q13, s13 = block_fp8.quantize_block_fp8(gate_up)
        q2, s2 = block_fp8.quantize_block_fp8(down)
        for i, expert in enumerate(block.experts):
            ib = inter // 128
            expert.gate_proj.weight.copy_(q13[i, :inter])
            expert.gate_proj.weight_scale_inv.copy_(s13[i, :ib])
            expert.up_proj.weight.copy_(q13[i, inter:])
            expert.up_proj.weight_scale_inv.copy_(s13[i, ib:])
            expert.down_proj.weight.copy_(q2[i])
            expert.down_proj.weight_scale_inv.copy_(s2[i])
