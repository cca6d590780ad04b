"""Configuration 3's measurement harness: a 12-layer DeBERTa-v3-base-shaped
encoder (hidden 768, 12 heads, FFN 3072, vocab 128100, one relative
embedding table shared by the layers with a LayerNorm, keys shared with the
relative projections, position buckets 256 / max relative positions 512)
around a disentangled-attention module, with the RTD discriminator head and
loss: BCE-with-logits of one logit per token against Bernoulli(0.15)
replaced-token labels, averaged over the active tokens.

The blocks keep the reference's structure and parameter names
(deberta_v2_native.py:115-165 self-output, :664-700 attention, :703-758 FFN,
:1036-1047 relative embeddings; rtd.py:550-626 head, :1129-1139 loss).  Two
parameters choose the implementation: the attention class (the fused
module on the GPU, or the oracle's restatement of the reference module on
the CPU) and ``fused_blocks`` (deberta_amd's fused row kernels around the
attention, or the plain torch layers below).  Both settings take the same
state dict.  This is a harness for the attention path and its neighbours,
not a model of this package.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch
from torch import nn

HIDDEN, HEADS, FFN, VOCAB, LAYERS = 768, 12, 3072, 128100, 12
BUCKETS, MAX_POS = 256, 512
EPS = 1e-7


def encoder_config(hidden: int = HIDDEN, heads: int = HEADS, ffn: int = FFN) -> SimpleNamespace:
    """The config of the harness (the reference's base preset: share_att_key,
    p2c|c2p, buckets 256, max_relative_positions -1 -> 512, LayerNorm eps
    1e-7, no dropout)."""
    return SimpleNamespace(
        hidden_size=hidden, num_attention_heads=heads, intermediate_size=ffn, share_att_key=True,
        pos_att_type="p2c|c2p", relative_attention=True, position_buckets=BUCKETS, max_relative_positions=-1,
        max_position_embeddings=MAX_POS, hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0,
        layer_norm_eps=EPS, norm_eps=EPS, hidden_act="gelu",
    )


# --- plain torch blocks (the reference's layers, deberta_v2_native.py:115-165, 703-758) ---------
class SelfOutput(nn.Module):
    def __init__(self, cfg, in_features=None):
        super().__init__()
        self.dense = nn.Linear(int(in_features or cfg.hidden_size), cfg.hidden_size)
        self.LayerNorm = nn.LayerNorm(cfg.hidden_size, eps=EPS)

    def forward(self, h, inp):
        return self.LayerNorm(self.dense(h) + inp)


class Output(SelfOutput):
    def __init__(self, cfg):
        super().__init__(cfg, in_features=cfg.intermediate_size)


class Intermediate(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.dense = nn.Linear(cfg.hidden_size, cfg.intermediate_size)

    def forward(self, h):
        return nn.functional.gelu(self.dense(h))


class RTDHead(nn.Module):
    """rtd.py:550-626 (LayerNorm head, "gelu", CLS context without a pairwise mask)."""

    def __init__(self, cfg):
        super().__init__()
        self.dense = nn.Linear(cfg.hidden_size, cfg.hidden_size)
        self.act = nn.GELU()
        self.norm = nn.LayerNorm(cfg.hidden_size, eps=EPS)
        self.classifier = nn.Linear(cfg.hidden_size, 1)

    def forward(self, h):
        x = self.norm(h + h[:, 0:1, :])
        return self.classifier(self.act(self.dense(x))).squeeze(-1)

    def forward_loss(self, h, labels, active=None):
        logits = self(h)
        return rtd_loss(logits, labels, active), logits


def rtd_loss(logits: torch.Tensor, labels: torch.Tensor, active=None) -> torch.Tensor:
    act = torch.ones_like(logits, dtype=torch.float32) if active is None else active.float()
    per = nn.functional.binary_cross_entropy_with_logits(logits.float(), labels.float(), reduction="none")
    return (per * act).sum() / act.sum().clamp(min=1.0)


class Attention(nn.Module):
    """DebertaV2Attention (deberta_v2_native.py:664-700): self + output."""

    def __init__(self, attn_cls, out_cls, cfg):
        super().__init__()
        self.self = attn_cls(cfg)
        self.output = out_cls(cfg)

    def forward(self, x, mask, rel_pos, rel):
        a, _ = self.self(x, mask, relative_pos=rel_pos, rel_embeddings=rel)
        return self.output(a, x)


class Layer(nn.Module):
    def __init__(self, attn_cls, cfg, fused_blocks: bool):
        super().__init__()
        if fused_blocks:
            from deberta_amd.blocks import FusedIntermediate, FusedOutput, FusedSelfOutput

            so, it, out = FusedSelfOutput, FusedIntermediate, FusedOutput
        else:
            so, it, out = SelfOutput, Intermediate, Output
        self.attention = Attention(attn_cls, so, cfg)
        self.intermediate = it(cfg)
        self.output = out(cfg)

    def forward(self, x, mask, rel_pos, rel):
        x = self.attention(x, mask, rel_pos, rel)
        return self.output(self.intermediate(x), x)


class Encoder(nn.Module):
    def __init__(self, attn_cls, layers: int = LAYERS, hidden: int = HIDDEN, heads: int = HEADS,
                 ffn: int = FFN, vocab: int = VOCAB, fused_blocks: bool = False):
        super().__init__()
        cfg = encoder_config(hidden, heads, ffn)
        self.fused_blocks = fused_blocks
        self.emb = nn.Embedding(vocab, hidden)
        self.emb_ln = nn.LayerNorm(hidden, eps=EPS)
        self.rel_embeddings = nn.Embedding(2 * BUCKETS, hidden)
        self.LayerNorm = nn.LayerNorm(hidden, eps=EPS)  # of the relative embeddings (norm_rel_ebd)
        self.layers = nn.ModuleList(Layer(attn_cls, cfg, fused_blocks) for _ in range(layers))
        if fused_blocks:
            from deberta_amd.blocks import FusedRTDHead

            self.head = FusedRTDHead(cfg)
        else:
            self.head = RTDHead(cfg)

    def hidden(self, ids, mask, rel_pos):
        x = self.emb_ln(self.emb(ids))
        if self.fused_blocks:
            from deberta_amd.blocks import fused_add_layer_norm

            rel = fused_add_layer_norm(self.rel_embeddings.weight, None, None, self.LayerNorm)
        else:
            rel = self.LayerNorm(self.rel_embeddings.weight)
        for layer in self.layers:
            x = layer(x, mask, rel_pos, rel)
        return x

    def forward(self, ids, mask, rel_pos):
        """Per-token logits (B, S)."""
        return self.head(self.hidden(ids, mask, rel_pos))

    def loss(self, ids, mask, rel_pos, labels, active=None):
        """(RTD loss, logits)."""
        return self.head.forward_loss(self.hidden(ids, mask, rel_pos), labels, active)


def init_weights(model: nn.Module, seed: int = 0) -> None:
    """N(0, 0.02) for matrices, zeros for biases, LayerNorm at (1, 0)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if prm.dim() > 1:
                prm.copy_(torch.randn(prm.shape, generator=g) * 0.02)
            elif "LayerNorm" in name or "emb_ln" in name or "norm" in name:
                prm.fill_(1.0 if name.endswith("weight") else 0.0)
            else:
                prm.zero_()


def synthetic_batch(batch: int, seq_len: int, vocab: int = VOCAB, seed: int = 0):
    """Token ids ~ U[0, vocab) and replaced-token labels ~ Bernoulli(0.15)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (batch, seq_len), generator=g)
    labels = (torch.rand(batch, seq_len, generator=g) < 0.15).float()
    return ids, labels
