"""A small randomly initialised action-expert block with the operator mix of the robotics
policies the reference studies (configs[1]-[4] shapes, scaled down): linear + bias, SiLU,
linear, HF-style RMSNorm (through ``mean``), grouped-query causal attention, a top-k SwiGLU
mixture of experts and a final action head.  Every sample is a token sequence [T, D]; the
model runs on the first ROCm GPU (CPU when there is none, for the harness's own tests).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


class _Block(torch.nn.Module):
    def __init__(self, d: int, hidden: int, heads: int, kv_heads: int, experts: int, inter: int,
                 top_k: int, actions: int, g: torch.Generator, dtype: torch.dtype):
        super().__init__()

        def w(*shape, scale=0.02):
            return torch.nn.Parameter((torch.randn(*shape, generator=g) * scale).to(dtype), requires_grad=False)

        self.heads, self.kv_heads, self.top_k = heads, kv_heads, top_k
        self.up = w(hidden, d)
        self.up_bias = w(hidden)
        self.down = w(d, hidden)
        self.norm_weight = torch.nn.Parameter(torch.ones(d, dtype=dtype), requires_grad=False)
        self.qkv = w((heads + 2 * kv_heads) * (d // heads), d)
        self.proj = w(d, d)
        self.router = w(experts, d, scale=1.0)
        self.gate_up = w(experts, d, 2 * inter)
        self.expert_down = w(experts, inter, d)
        self.head = w(actions, d)

    def rms_norm(self, x: torch.Tensor) -> torch.Tensor:
        var = x.float().pow(2).mean(-1, keepdim=True)
        return (x.float() * torch.rsqrt(var + 1e-6)).to(x.dtype) * self.norm_weight

    def forward(self, x: torch.Tensor) -> dict[str, torch.Tensor]:
        from batch_invariant_ops import deterministic_token_choice_moe

        b, t, d = x.shape
        h = x + F.linear(F.silu(F.linear(x, self.up, self.up_bias)), self.down)
        h = self.rms_norm(h)
        hd = d // self.heads
        q, k, v = F.linear(h, self.qkv).split([self.heads * hd, self.kv_heads * hd, self.kv_heads * hd], -1)
        q = q.view(b, t, self.heads, hd).transpose(1, 2)
        k = k.view(b, t, self.kv_heads, hd).transpose(1, 2)
        v = v.view(b, t, self.kv_heads, hd).transpose(1, 2)
        att = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        h = h + F.linear(att.transpose(1, 2).reshape(b, t, d), self.proj)
        h = self.rms_norm(h)
        tokens = h.reshape(b * t, d)
        probs = torch.softmax(F.linear(tokens, self.router).float(), dim=-1)
        weights, experts = torch.topk(probs, self.top_k, dim=-1)
        inter = self.expert_down.shape[1]
        if tokens.is_cuda:
            moe = deterministic_token_choice_moe(
                tokens, weights, experts,
                self.gate_up[..., :inter].transpose(1, 2), self.gate_up[..., inter:].transpose(1, 2),
                self.expert_down.transpose(1, 2))
        else:  # CPU: the same formula with stock ops (the harness's own tests)
            moe = torch.zeros_like(tokens)
            for s in range(self.top_k):
                e = experts[:, s]
                g_ = torch.einsum("td,tdi->ti", tokens, self.gate_up[e, :, :inter])
                u_ = torch.einsum("td,tdi->ti", tokens, self.gate_up[e, :, inter:])
                y = torch.einsum("ti,tid->td", F.silu(g_) * u_, self.expert_down[e])
                moe = moe + y * weights[:, s:s + 1].to(y.dtype)
        h = h + moe.view(b, t, d)
        actions = F.linear(h[:, -8:], self.head)
        return {"actions": actions, "router_top_k": experts.view(b, t, self.top_k),
                "pooled": torch.linalg.vector_norm(h, dim=-1)}


# Sizes: "small" for quick checks; "vla" uses the action-expert widths of configs[1]-[2]
# (D 2048, MLP 8192, 16 query / 4 KV heads of 128, 256 tokens per sample).
PRESETS = {
    "small": dict(tokens=64, d=256, hidden=1024, heads=8, kv_heads=2, experts=8, inter=128, top_k=2),
    "vla": dict(tokens=256, d=2048, hidden=8192, heads=16, kv_heads=4, experts=8, inter=768, top_k=2),
}


class SyntheticVLAAdapter:
    """Harness adapter around ``_Block``; samples are seeded token sequences [T, D]."""

    name = "synthetic_vla"

    def __init__(self, tokens: int = 64, d: int = 256, hidden: int = 1024, heads: int = 8,
                 kv_heads: int = 2, experts: int = 8, inter: int = 128, top_k: int = 2,
                 actions: int = 7, dtype: torch.dtype = torch.bfloat16, device: str | None = None):
        self.tokens, self.d = tokens, d
        self.cfg = (d, hidden, heads, kv_heads, experts, inter, top_k, actions)
        self.dtype = dtype
        self.device = device or ("cuda" if torch.cuda.is_available() else "cpu")

    @classmethod
    def preset(cls, name: str, **overrides) -> "SyntheticVLAAdapter":
        return cls(**{**PRESETS[name], **overrides})

    def load_model(self) -> torch.nn.Module:
        g = torch.Generator().manual_seed(1234)
        return _Block(*self.cfg, g=g, dtype=self.dtype).to(self.device)

    def load_example_inputs(self, count: int) -> list[dict[str, torch.Tensor]]:
        g = torch.Generator().manual_seed(4321)
        return [{"x": torch.randn(self.tokens, self.d, generator=g).to(self.dtype).to(self.device)}
                for _ in range(count)]

    def run_model(self, model: torch.nn.Module, batch: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
        return model(batch["x"])

    def extract_robot_output(self, output: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
        return output
