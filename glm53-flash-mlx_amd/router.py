"""FP32 top-k router (patch.py:131-142 ``Float32Gate`` of the reference).

logits = x_f32 @ W_f32^T, sigma = sigmoid(logits), choice = sigma + bias
(``e_score_correction_bias``), ids = top_k(choice) ordered by (choice desc,
expert id asc), weights = sigma[ids] normalised when ``norm_topk_prob`` and
multiplied by ``routed_scaling_factor``.  The selection rule is the
DeepSeek-V3 auxiliary-loss-free rule that mlx-vlm's
``dsv32.group_expert_select`` implements: with n_group > 1 the experts form
n_group groups of consecutive ids, each scored by the FP32 sum of its two
largest biased scores, and the biased scores outside the topk_group best
groups become 0.0 before the top-k.  The slot order and the order of equal
group scores (MLX leaves argpartition order unspecified) are this build's
documented tie policy: (choice desc, expert id asc), lower group index
kept.  One token runs a one-workgroup-per-logit kernel, several tokens an
LDS-tiled BF16-MFMA GEMM over the exact three-way BF16 split of the FP32
weights; then a wavefront-per-token top-k.
"""

from __future__ import annotations

import torch

from . import _native as N
from . import ops as _ops  # noqa: F401  (registers the glm53 custom ops)


class Float32Gate(torch.nn.Module):
    def __init__(self, weight: torch.Tensor, bias: torch.Tensor, *, top_k: int = 8,
                 routed_scaling_factor: float = 1.0, norm_topk_prob: bool = True, n_group: int = 1,
                 topk_group: int = 1):
        super().__init__()
        if weight.dtype != torch.float32 or weight.dim() != 2:
            raise ValueError("router weight must be a 2-D float32 [experts, hidden] tensor")
        if bias.dtype != torch.float32 or bias.shape != (weight.shape[0],):
            raise ValueError("e_score_correction_bias must be float32 [experts]")
        check_groups(weight.shape[0], int(top_k), int(n_group), int(topk_group))
        self.register_buffer("weight", weight.contiguous())
        self.register_buffer("e_score_correction_bias", bias.contiguous())
        self.top_k = int(top_k)
        self.routed_scaling_factor = float(routed_scaling_factor)
        self.norm_topk_prob = bool(norm_topk_prob)
        self.n_group = int(n_group)
        self.topk_group = int(topk_group)

    @property
    def n_routed_experts(self) -> int:
        return int(self.weight.shape[0])

    def as_c_struct(self) -> N.Router:
        return N.Router(self.weight.data_ptr(), self.e_score_correction_bias.data_ptr(), self.weight.shape[0],
                        self.weight.shape[1], self.top_k, self.routed_scaling_factor, int(self.norm_topk_prob),
                        self.n_group, self.topk_group)

    def forward(self, x):
        N.require_device(x, self.weight)
        if x.dtype != torch.bfloat16:
            raise ValueError(f"router input must be bfloat16, got {x.dtype}")
        hidden = self.weight.shape[1]
        if x.shape[-1] != hidden:
            raise ValueError(f"input width {x.shape[-1]} != router width {hidden}")
        return torch.ops.glm53.router_topk(x, self.weight, self.e_score_correction_bias, self.top_k,
                                           self.routed_scaling_factor, self.norm_topk_prob, self.n_group,
                                           self.topk_group)


def check_groups(experts: int, top_k: int, n_group: int, topk_group: int) -> None:
    """ValueError unless (n_group, topk_group) is a selection the kernels take:
    1 <= topk_group <= n_group <= 64, n_group dividing the experts into
    groups of two or more, and top_k experts available in the kept groups."""
    if not 1 <= topk_group <= n_group <= 64:
        raise ValueError(f"need 1 <= topk_group <= n_group <= 64, got n_group={n_group}, topk_group={topk_group}")
    if n_group > 1:
        if experts % n_group or experts // n_group < 2:
            raise ValueError(f"n_group={n_group} must split {experts} experts into equal groups of two or more")
        if top_k > topk_group * (experts // n_group):
            raise ValueError(f"top_k={top_k} exceeds the {topk_group * (experts // n_group)} experts of the kept groups")


def native_router_topk(x, weight, bias, top_k: int, routed_scaling_factor: float, norm_topk_prob: bool,
                       n_group: int = 1, topk_group: int = 1):
    """The native call behind the glm53::router_topk op."""
    hidden = weight.shape[1]
    flat = x.reshape(-1, hidden).contiguous()
    tokens = flat.shape[0]
    ids = torch.empty((tokens, top_k), dtype=torch.int32, device=x.device)
    scores = torch.empty((tokens, top_k), dtype=torch.float32, device=x.device)
    lib = N.lib()
    ws_bytes = lib.glm53_router_workspace_bytes(tokens, hidden, weight.shape[0])
    ws = N.workspace(ws_bytes, x.device)
    router = N.Router(weight.data_ptr(), bias.data_ptr(), weight.shape[0], hidden, top_k, float(routed_scaling_factor),
                      int(norm_topk_prob), int(n_group), int(topk_group))
    N.check(lib.glm53_router_topk(N.ctypes.byref(router), N.ptr(flat), tokens, N.ptr(ids), N.ptr(scores),
                                  N.ptr(ws), ws_bytes, N.stream_handle(x.device)))
    lead = x.shape[:-1]
    return ids.reshape(*lead, top_k), scores.reshape(*lead, top_k)
