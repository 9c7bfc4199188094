"""Small seeded transformer-shaped models for loader tests (module names follow the HF
decoder layout the reference's loader walks: model.layers[i].self_attn.{q,k,v,o}_proj and
mlp.{gate,up,down}_proj, src/kernels/quantization.py:480-514)."""

import torch
import torch.nn as nn
import torch.nn.functional as F


class Attn(nn.Module):
    def __init__(self, h, bias):
        super().__init__()
        self.q_proj = nn.Linear(h, h, bias=bias)
        self.k_proj = nn.Linear(h, h, bias=bias)
        self.v_proj = nn.Linear(h, h, bias=bias)
        self.o_proj = nn.Linear(h, h, bias=False)

    def forward(self, x):
        q, k, v = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        p = torch.softmax(q @ k.transpose(-1, -2) / q.shape[-1] ** 0.5, dim=-1)
        return self.o_proj(p @ v)


class Mlp(nn.Module):
    def __init__(self, h, inter, bias):
        super().__init__()
        self.gate_proj = nn.Linear(h, inter, bias=bias)
        self.up_proj = nn.Linear(h, inter, bias=bias)
        self.down_proj = nn.Linear(inter, h, bias=bias)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class Block(nn.Module):
    def __init__(self, h, inter, attn_bias, mlp_bias):
        super().__init__()
        self.self_attn = Attn(h, attn_bias)
        self.mlp = Mlp(h, inter, mlp_bias)

    def forward(self, x):
        x = x + self.self_attn(x)
        return x + self.mlp(x)


class Body(nn.Module):
    def __init__(self, h, n_layers, attn_bias, mlp_bias):
        super().__init__()
        self.layers = nn.ModuleList(Block(h, 2 * h, attn_bias, mlp_bias) for _ in range(n_layers))

    def forward(self, x):
        for blk in self.layers:
            x = blk(x)
        return x


class TinyCausalLM(nn.Module):
    def __init__(self, h=64, n_layers=2, vocab=256, attn_bias=True, mlp_bias=False):
        super().__init__()
        self.model = Body(h, n_layers, attn_bias, mlp_bias)
        self.lm_head = nn.Linear(h, vocab, bias=False)

    def forward(self, x):
        return self.lm_head(self.model(x))


def seeded_model(seed=42, **kw):
    torch.manual_seed(seed)
    m = TinyCausalLM(**kw)
    m.eval()
    return m
