"""The tiny decoder LM workload shared by the GPU test and the fixture
generator: a 4-layer GPT-style decoder (d 256, 4 heads, MLP 1024, vocab 512,
seq 128; 3,323,392 parameters in 52 tensors, LM head tied to the token
embedding), the layout of minispeed's examples/train_lm.py:62-115.

Initialisation (fixed here, both sides use it): LayerNorm weights 1, every
other 1-D tensor 0, matrices N(0, 0.02), drawn in parameter order from
``torch.manual_seed(seed)`` on the CPU.  Token batches are uniform ids from a
seeded CPU generator, so the reference's CPU run and the GPU run see the
same bits.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

VOCAB, SEQ, D, LAYERS, HEADS, MICRO = 512, 128, 256, 4, 4, 8


class Block(nn.Module):
    def __init__(self, d, heads):
        super().__init__()
        self.heads = heads
        self.ln1 = nn.LayerNorm(d)
        self.qkv = nn.Linear(d, 3 * d)
        self.proj = nn.Linear(d, d)
        self.ln2 = nn.LayerNorm(d)
        self.fc = nn.Linear(d, 4 * d)
        self.fc2 = nn.Linear(4 * d, d)

    def forward(self, x):
        b, t, c = x.shape
        q, k, v = self.qkv(self.ln1(x)).chunk(3, dim=-1)
        q, k, v = (z.view(b, t, self.heads, c // self.heads).transpose(1, 2) for z in (q, k, v))
        att = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + self.proj(att.transpose(1, 2).contiguous().view(b, t, c))
        return x + self.fc2(F.gelu(self.fc(self.ln2(x))))


class TinyLM(nn.Module):
    def __init__(self, vocab=VOCAB, block=SEQ, d=D, layers=LAYERS, heads=HEADS):
        super().__init__()
        self.wte = nn.Embedding(vocab, d)
        self.wpe = nn.Embedding(block, d)
        self.blocks = nn.ModuleList(Block(d, heads) for _ in range(layers))
        self.ln_f = nn.LayerNorm(d)
        self.head = nn.Linear(d, vocab, bias=False)
        self.head.weight = self.wte.weight
        with torch.no_grad():
            for name, p in self.named_parameters():
                if name.endswith("ln1.weight") or name.endswith("ln2.weight") or name == "ln_f.weight":
                    p.fill_(1.0)
                elif p.dim() == 1:
                    p.zero_()
                else:
                    p.normal_(0.0, 0.02)

    def forward(self, idx):
        t = idx.shape[1]
        x = self.wte(idx) + self.wpe(torch.arange(t, device=idx.device))
        for blk in self.blocks:
            x = blk(x)
        return self.head(self.ln_f(x))


def build(seed: int = 0) -> TinyLM:
    """The model on the CPU, initialised from ``seed``."""
    torch.manual_seed(seed)
    return TinyLM()


def batches(steps: int, seed: int = 1) -> torch.Tensor:
    """``[steps, MICRO, SEQ + 1]`` int64 token ids (CPU)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, VOCAB, (steps, MICRO, SEQ + 1), generator=g)


def loss_fn(logits: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    return F.cross_entropy(logits.reshape(-1, VOCAB).float(), idx[:, 1:].reshape(-1))


CONFIG = {"train_micro_batch_size_per_gpu": MICRO, "gradient_accumulation_steps": 1,
          "gradient_clipping": 1.0, "dtype": "fp32",
          "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "betas": [0.9, 0.999], "eps": 1e-8,
                                                     "weight_decay": 0.01}},
          "zero_optimization": {"stage": 0}, "steps_per_print": 1000}
