"""Eager torch-CPU restatement of the reference's blocks around the attention
— TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Each function names the reference lines it restates (pszemraj/deberta,
paths relative to src/deberta/).  Parameter names follow the reference
modules, so the fused modules of deberta_amd.blocks load the same state
dicts.
"""

from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


# --- modeling/deberta_v2_native.py:115-165 (SelfOutput), 733-758 (Output) ----
class OutputResidualNorm(nn.Module):
    """dense -> dropout -> LayerNorm(x + input_tensor) (_apply_output_residual_norm, :146-165)."""

    def __init__(self, config: Any, in_features: Optional[int] = None) -> None:
        super().__init__()
        hidden = int(config.hidden_size)
        self.dense = nn.Linear(int(in_features or hidden), hidden)
        self.LayerNorm = nn.LayerNorm(hidden, eps=float(getattr(config, "layer_norm_eps", 1e-7)))
        self.dropout = nn.Dropout(float(getattr(config, "hidden_dropout_prob", 0.0)))

    def forward(self, hidden_states: torch.Tensor, input_tensor: torch.Tensor) -> torch.Tensor:
        x = self.dense(hidden_states)
        x = self.dropout(x)
        return self.LayerNorm(x + input_tensor)


# --- modeling/deberta_v2_native.py:703-730 (Intermediate, hidden_act "gelu") -
class Intermediate(nn.Module):
    def __init__(self, config: Any) -> None:
        super().__init__()
        self.dense = nn.Linear(int(config.hidden_size), int(config.intermediate_size))

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return F.gelu(self.dense(hidden_states))


# --- modeling/rtd.py:550-626 (RTDHead, LayerNorm head, "gelu") ---------------
class RTDHead(nn.Module):
    def __init__(self, config: Any) -> None:
        super().__init__()
        hidden = int(config.hidden_size)
        self.dense = nn.Linear(hidden, hidden)
        self.act = nn.GELU()
        eps = float(getattr(config, "norm_eps", getattr(config, "layer_norm_eps", 1e-6)))
        self.norm = nn.LayerNorm(hidden, eps=eps)
        self.classifier = nn.Linear(hidden, 1)

    @staticmethod
    def use_global_cls_context(attention_mask: Optional[torch.Tensor]) -> bool:
        if attention_mask is None:
            return True
        mask = attention_mask
        if mask.ndim == 4:
            mask = mask[:, 0] if mask.shape[1] == 1 else mask.any(dim=1)
        if mask.ndim == 3 and mask.shape[-2] != 1:
            return False
        return True

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.use_global_cls_context(attention_mask):
            ctx = hidden_states[:, 0:1, :]
            x = self.norm(hidden_states + ctx)
        else:
            x = self.norm(hidden_states)
        x = self.dense(x)
        x = self.act(x)
        return self.classifier(x).squeeze(-1)


# --- modeling/rtd.py:1129-1139 (discriminator loss) ---------------------------
def discriminator_loss(logits: torch.Tensor, labels: torch.Tensor, active: Optional[torch.Tensor]) -> torch.Tensor:
    act = torch.ones_like(logits, dtype=torch.float32) if active is None else active.to(torch.float32)
    denom = act.sum().clamp(min=1.0)
    per_token = F.binary_cross_entropy_with_logits(logits.float(), labels.float(), reduction="none")
    return (per_token * act).sum() / denom


# --- modeling/deberta_v2_native.py:1036-1047 (get_rel_embedding, layer_norm) --
class RelativeEmbeddings(nn.Module):
    def __init__(self, config: Any) -> None:
        super().__init__()
        hidden = int(config.hidden_size)
        buckets = int(getattr(config, "position_buckets", -1))
        max_rel = int(getattr(config, "max_relative_positions", -1))
        if max_rel < 1:
            max_rel = int(config.max_position_embeddings)
        pos_ebd = buckets if buckets > 0 else max_rel
        self.rel_embeddings = nn.Embedding(pos_ebd * 2, hidden)
        self.LayerNorm = nn.LayerNorm(hidden, eps=float(getattr(config, "layer_norm_eps", 1e-7)), elementwise_affine=True)

    def forward(self) -> torch.Tensor:
        return self.LayerNorm(self.rel_embeddings.weight)
