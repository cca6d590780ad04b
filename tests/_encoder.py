"""Configuration 3's measurement harness: a 12-layer DeBERTa-v3-base-shaped
encoder (hidden 768, 12 heads, FFN 3072, vocab 128100, one relative
embedding table shared by the layers with a LayerNorm, keys shared with the
relative projections, position buckets 256 / max relative positions 512)
around a disentangled-attention module, with an RTD-style discriminator
loss: BCE-with-logits of one logit per token against Bernoulli(0.15)
replaced-token labels.

It is a harness for the attention path, not a model of this package: the
blocks around the attention are plain torch layers shaped like the
reference's (deberta_v2_native.py:115-165 self-output, :703-758 FFN,
rtd.py:552-626 head and loss).  The attention class is a parameter, so the
same encoder runs with the fused module on the GPU and with the oracle's
restatement of the reference module on the CPU.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch
from torch import nn

HIDDEN, HEADS, FFN, VOCAB, LAYERS = 768, 12, 3072, 128100, 12
BUCKETS, MAX_POS = 256, 512


def encoder_config(hidden: int = HIDDEN, heads: int = HEADS) -> SimpleNamespace:
    """The attention config of the harness (the reference's base preset:
    share_att_key, p2c|c2p, buckets 256, max_relative_positions -1 -> 512)."""
    return SimpleNamespace(
        hidden_size=hidden, num_attention_heads=heads, share_att_key=True, pos_att_type="p2c|c2p",
        relative_attention=True, position_buckets=BUCKETS, max_relative_positions=-1,
        max_position_embeddings=MAX_POS, hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0,
    )


class Layer(nn.Module):
    def __init__(self, attn_cls, cfg, hidden: int, ffn: int):
        super().__init__()
        self.attn = attn_cls(cfg)
        self.out = nn.Linear(hidden, hidden)
        self.ln1 = nn.LayerNorm(hidden, eps=1e-7)
        self.up, self.down = nn.Linear(hidden, ffn), nn.Linear(ffn, hidden)
        self.ln2 = nn.LayerNorm(hidden, eps=1e-7)

    def forward(self, x, mask, rel_pos, rel):
        a, _ = self.attn(x, mask, relative_pos=rel_pos, rel_embeddings=rel)
        x = self.ln1(self.out(a) + x)
        return self.ln2(self.down(nn.functional.gelu(self.up(x))) + x)


class Encoder(nn.Module):
    def __init__(self, attn_cls, layers: int = LAYERS, hidden: int = HIDDEN, heads: int = HEADS,
                 ffn: int = FFN, vocab: int = VOCAB):
        super().__init__()
        cfg = encoder_config(hidden, heads)
        self.emb = nn.Embedding(vocab, hidden)
        self.emb_ln = nn.LayerNorm(hidden, eps=1e-7)
        self.rel = nn.Parameter(torch.empty(2 * BUCKETS, hidden))
        self.rel_ln = nn.LayerNorm(hidden, eps=1e-7)
        self.layers = nn.ModuleList(Layer(attn_cls, cfg, hidden, ffn) for _ in range(layers))
        self.head = nn.Sequential(nn.Linear(hidden, hidden), nn.GELU(), nn.LayerNorm(hidden, eps=1e-7), nn.Linear(hidden, 1))

    def forward(self, ids, mask, rel_pos):
        x = self.emb_ln(self.emb(ids))
        rel = self.rel_ln(self.rel)
        for layer in self.layers:
            x = layer(x, mask, rel_pos, rel)
        return self.head(x).squeeze(-1)


def init_weights(model: nn.Module, seed: int = 0) -> None:
    """N(0, 0.02) for matrices, zeros for biases, LayerNorm at (1, 0)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if prm.dim() > 1:
                prm.copy_(torch.randn(prm.shape, generator=g) * 0.02)
            elif "ln" not in name and "head.2" not in name:
                prm.zero_()


def synthetic_batch(batch: int, seq_len: int, vocab: int = VOCAB, seed: int = 0):
    """Token ids ~ U[0, vocab) and replaced-token labels ~ Bernoulli(0.15)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (batch, seq_len), generator=g)
    labels = (torch.rand(batch, seq_len, generator=g) < 0.15).float()
    return ids, labels


def rtd_loss(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    return nn.functional.binary_cross_entropy_with_logits(logits.float(), labels)
