"""Stand-ins for the diffusers Attention module in processor tests."""
import torch
import torch.nn as nn


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        return x * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + self.eps).to(x.dtype) * self.weight


class StubAttention(nn.Module):
    """The diffusers Attention members the processors touch."""

    def __init__(self, dim=64, heads=2, added_kv=False, added_q=False, norm_shape=None):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = (nn.Linear(dim, dim) for _ in range(3))
        ns = norm_shape or dim
        self.norm_q, self.norm_k = RMSNorm(ns), RMSNorm(ns)
        self.add_k_proj = nn.Linear(dim, dim) if added_kv else None
        self.add_v_proj = nn.Linear(dim, dim) if added_kv else None
        self.norm_added_k = RMSNorm(ns) if (added_kv or added_q) else None
        self.add_q_proj = nn.Linear(dim, dim) if added_q else None
        if added_q:
            self.add_k_proj = nn.Linear(dim, dim)
            self.add_v_proj = nn.Linear(dim, dim)
        self.norm_added_q = RMSNorm(ns) if added_q else None
        self.to_out = nn.ModuleList([nn.Linear(dim, dim), nn.Dropout(0.0)])
        self.to_add_out = nn.Linear(dim, dim) if added_q else None
        self.processor = None

    def get_processor(self):
        return self.processor

    def set_processor(self, p):
        self.processor = p
