"""The tiny decoder LM workload end to end on the GPU.

A 4-layer GPT-style decoder (d 256, 4 heads, MLP 1024, vocab 512, seq 128;
3,323,392 parameters in 52 tensors, LM head tied to the token embedding, the
layout of minispeed's examples/train_lm.py:62-115), random N(0,0.02) init,
micro-batch 8 of uniform random token ids, fp32, ZeRO 0, AdamW lr 1e-3
betas (0.9,0.999) eps 1e-8 wd 0.01, clip 1.0, 20 boundaries.

Forward and backward run through torch autograd on the GPU; every boundary
is checked against the oracle started from the GPU's own state with the
gradients autograd produced (copied before ``engine.step`` releases them).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

import minispeed_amd as ms
from minispeed_amd.workloads import numel, shapes_of
from oracle import boundary as ob
from oracle import recipe
from tests.helpers import master_step_within_ulps

pytestmark = pytest.mark.gpu
DEV = "cuda"


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
    def __init__(self, vocab=512, block=128, d=256, layers=4, heads=4):
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


def test_tiny_lm_trains_through_the_engine_and_matches_the_oracle_each_step():
    torch.manual_seed(0)
    model = TinyLM().to(DEV)
    shapes = [tuple(p.shape) for p in model.parameters()]
    assert shapes == shapes_of("tiny-lm-3.3m") and numel(shapes) == 3_323_392
    cfg = {"train_micro_batch_size_per_gpu": 8, "gradient_accumulation_steps": 1,
           "gradient_clipping": 1.0, "dtype": "fp32",
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "betas": [0.9, 0.999], "eps": 1e-8,
                                                      "weight_decay": 0.01}},
           "zero_optimization": {"stage": 0}}
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()), config=cfg)
    params = list(model.parameters())
    ref_params = [nn.Parameter(p.detach().cpu().clone()) for p in params]
    ref = ob.Engine([ref_params], [{"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8,
                                    "weight_decay": 0.01}], dtype="fp32", zero_stage=0, clip=1.0,
                    scheduler_params={"warmup_max_lr": 1e-3})
    gen = torch.Generator(device=DEV).manual_seed(1)
    g = engine.flat_groups[0]
    losses = []
    for step in range(20):
        idx = torch.randint(0, 512, (8, 129), generator=gen, device=DEV)
        logits = engine(idx[:, :-1])
        loss = F.cross_entropy(logits.reshape(-1, 512), idx[:, 1:].reshape(-1))
        losses.append(float(loss.detach()))
        engine.backward(loss)
        grads = [p.grad.detach().cpu().clone() for p in params]
        before = g.data.detach().cpu()
        st = engine.optimizer.state[0]
        ref.load_state([before], [st["exp_avg"].cpu()], [st["exp_avg_sq"].cpu()], [st["step"]],
                       (1.0, 0, 0), engine.lr_scheduler.last_epoch,
                       [pg["lr"] for pg in engine.optimizer.param_groups])
        for rp, gr in zip(ref_params, grads):
            rp.grad = gr
        ref.micro_steps += 1
        assert engine.step() is True and ref.step() is True
        assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
        _, _, coef = recipe.clip_coef(np.float32(ref.grad_norm), 1.0)
        same = np.float32(engine.last_boundary.coef) == np.float32(coef)
        ok, worst = master_step_within_ulps(before.numpy(), g.data.cpu().numpy(),
                                            ref.groups[0].data.numpy(), 2.0 if same else 4.0)
        assert ok, (step, worst)
        if same:
            np.testing.assert_array_equal(st["exp_avg"].cpu().numpy(), ref.state[0]["exp_avg"].numpy())
            np.testing.assert_array_equal(st["exp_avg_sq"].cpu().numpy(),
                                          ref.state[0]["exp_avg_sq"].numpy())
        # fp32 model: the parameters are the masters
        for (off, p), n in zip(g._offsets, g._numels):
            assert torch.equal(p.detach().reshape(-1), g.data[off:off + n])
    assert engine.global_steps == 20
    assert np.mean(losses[-5:]) < np.mean(losses[:5])
