"""Ragged parameter lists of the benchmark models, in parameter order.

GPT shapes follow ``TinyGPT`` of minispeed's examples/train_lm.py:62-115
(token and position embeddings, 12 tensors per block, final LayerNorm; the
LM head is tied to the token embedding, so it is not a separate tensor).
Llama-3-8B shapes follow the usual decoder layout (embedding, per layer
q/k/v/o, gate/up/down, two RMSNorm weights, final norm, untied LM head).
"""

from __future__ import annotations

from typing import Dict, List, Tuple

Shape = Tuple[int, ...]


def gpt_shapes(n_layer: int, d: int, vocab: int, block: int) -> List[Shape]:
    shapes: List[Shape] = [(vocab, d), (block, d)]
    for _ in range(n_layer):
        shapes += [
            (d,), (d,),                  # ln1
            (3 * d, d), (3 * d,),        # attn.qkv
            (d, d), (d,),                # attn.proj
            (d,), (d,),                  # ln2
            (4 * d, d), (4 * d,),        # mlp fc
            (d, 4 * d), (d,),            # mlp proj
        ]
    shapes += [(d,), (d,)]               # ln_f
    return shapes


def llama3_8b_shapes() -> List[Shape]:
    d, kv, ffn, vocab = 4096, 1024, 14336, 128256
    shapes: List[Shape] = [(vocab, d)]
    for _ in range(32):
        shapes += [(d, d), (kv, d), (kv, d), (d, d), (ffn, d), (ffn, d), (d, ffn), (d,), (d,)]
    shapes += [(d,), (vocab, d)]
    return shapes


WORKLOADS: Dict[str, dict] = {
    "tiny-lm-3.3m": dict(shapes=lambda: gpt_shapes(4, 256, 512, 128),
                         desc="tiny GPT decoder (4 layers, d 256, vocab 512, seq 128)"),
    "gpt2-124m": dict(shapes=lambda: gpt_shapes(12, 768, 50257, 1024),
                      desc="GPT-2-small buffer (12 layers, d 768, vocab 50257)"),
    "gpt-350m": dict(shapes=lambda: gpt_shapes(24, 1024, 50257, 1024),
                     desc="350M GPT buffer (24 layers, d 1024, vocab 50257)"),
    "gpt-1.3b": dict(shapes=lambda: gpt_shapes(24, 2048, 50257, 2048),
                     desc="1.3B GPT buffer (24 layers, d 2048, vocab 50257, seq 2048)"),
    # the same after a 3-element tensor: flat layouts pack tensors back to
    # back, so every later gradient and model copy starts 3 elements off the
    # 16-byte grid of the flat space (as after an odd-sized vocabulary bias)
    "gpt-1.3b-shift3": dict(shapes=lambda: [(3,)] + gpt_shapes(24, 2048, 50257, 2048),
                            desc="1.3B GPT buffer after a 3-element tensor (every later "
                                 "tensor off the flat space's 16-byte grid)"),
    "llama3-8b": dict(shapes=llama3_8b_shapes,
                      desc="Llama-3-8B (32 layers, d 4096, GQA 32q/8kv, FFN 14336, vocab 128256)"),
}


def shapes_of(name: str) -> List[Shape]:
    return WORKLOADS[name]["shapes"]()


def numel(shapes: List[Shape]) -> int:
    total = 0
    for s in shapes:
        n = 1
        for x in s:
            n *= x
        total += n
    return total
