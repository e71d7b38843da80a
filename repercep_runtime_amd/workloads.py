"""The BASELINE configurations of the FP8 hot path and their seeded synthetic inputs.

Inputs follow one recipe so the GPU run and any CPU check see identical
tensors: a ``torch.Generator`` seeded per config draws fp32 N(0, 1) in the
order Q, K, V (then weights), each rounded to bf16.  Seed 0 for attention,
seed 1 for the GEMM.  The Cosmos config applies a per-head RMSNorm over D
(eps 1e-6, unit weight, fp32 math) to Q and K before quantization, as the
Cosmos attention processor does ahead of dispatch.

FLOP counts are the algorithmic ones (4*B*H*Sq*Skv*D for non-causal
attention: two matmuls of 2 FLOP per multiply-add; for the shared-prefix
mask only visible (query, key) pairs count), and the quantizer's traffic is
5 bytes per element (2 B read for amax, 2 B read + 1 B write to quantize).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

QUANT_BYTES_PER_ELEM = 5


@dataclass(frozen=True)
class AttnConfig:
    name: str
    B: int
    H: int
    Sq: int
    Skv: int
    D: int
    causal: bool = False
    rmsnorm_qk: bool = False
    prefix: int | None = None   # shared-prefix candidate mask
    suffix: int | None = None
    seed: int = 0
    description: str = ""

    def visible_pairs_per_head(self) -> int:
        if self.prefix is not None:
            assert self.suffix is not None
            n_cand = self.Sq // self.suffix
            own = self.suffix * (self.suffix + 1) // 2
            return n_cand * (self.suffix * self.prefix + own)
        if self.causal:
            # kv <= q with queries and keys aligned at 0
            return sum(min(q + 1, self.Skv) for q in range(self.Sq))
        return self.Sq * self.Skv

    @property
    def flops(self) -> float:
        return 4.0 * self.B * self.H * self.visible_pairs_per_head() * self.D

    @property
    def quant_elems(self) -> int:
        return self.B * self.H * (self.Sq + 2 * self.Skv) * self.D


@dataclass(frozen=True)
class GemmConfig:
    name: str
    M: int
    K: int
    N: int
    w_std: float = 0.02
    seed: int = 1

    @property
    def flops(self) -> float:
        return 2.0 * self.M * self.N * self.K


C1 = AttnConfig("c1_cpu_runnable", 1, 8, 1024, 1024, 64,
                description="FP8 flash-attn fwd, CPU-runnable reference case")
C2 = AttnConfig("c2_cosmos_self", 1, 32, 56320, 56320, 128, rmsnorm_qk=True,
                description="Cosmos-7B DiT self-attention, 16x44x80 latent grid")
C3_SELF = AttnConfig("c3_wan_self", 1, 40, 75600, 75600, 128,
                     description="Wan-2.2-A14B self-attention, 21x45x80 latent grid")
C3_CROSS = AttnConfig("c3_wan_cross", 1, 40, 75600, 512, 128,
                      description="Wan-2.2-A14B cross-attention to 512 text tokens")
C5 = AttnConfig("c5_shared_prefix", 1, 32, 128, 640, 128, prefix=512, suffix=8,
                description="token-VLA candidate decode: 512 shared prefix + 16 x 8 suffix")
C4 = GemmConfig("c4_wan_ffn_up", 75600, 5120, 13824)

ATTN_CONFIGS = {c.name: c for c in (C1, C2, C3_SELF, C3_CROSS, C5)}


def _randn_bf16(gen: torch.Generator, shape: tuple[int, ...], device: torch.device,
                std: float = 1.0) -> torch.Tensor:
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if std != 1.0:
        x.mul_(std)
    return x.to(torch.bfloat16)


def rmsnorm_heads(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Per-(b, h, s) RMSNorm over D with unit weight, fp32 math, bf16 result."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)).to(torch.bfloat16)


def attn_inputs(cfg: AttnConfig, device: str | torch.device = "cpu",
                heads: int | None = None, normalize: bool = True
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Seeded (Q, K, V) bf16 tensors in (B, H, S, D) layout on ``device``.

    ``heads`` limits H (the first heads of the same stream are *not*
    reproduced by a smaller H; use it only for standalone samples).
    ``normalize=False`` leaves out the config's QK RMSNorm (for a caller
    that fuses it into the quantizer).
    """
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(cfg.seed)
    H = cfg.H if heads is None else heads
    q = _randn_bf16(gen, (cfg.B, H, cfg.Sq, cfg.D), dev)
    k = _randn_bf16(gen, (cfg.B, H, cfg.Skv, cfg.D), dev)
    v = _randn_bf16(gen, (cfg.B, H, cfg.Skv, cfg.D), dev)
    if cfg.rmsnorm_qk and normalize:
        q = rmsnorm_heads(q)
        k = rmsnorm_heads(k)
    return q, k, v


def gemm_inputs(cfg: GemmConfig, device: str | torch.device = "cpu",
                rows: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Seeded activations A (M, K) ~ N(0, 1) and weights W (K, N) ~ N(0, w_std), bf16."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(cfg.seed)
    M = cfg.M if rows is None else rows
    a = _randn_bf16(gen, (M, cfg.K), dev)
    w = _randn_bf16(gen, (cfg.K, cfg.N), dev, std=cfg.w_std)
    return a, w
