"""Spikformer (spiking vision transformer) for the attention workload.

The reference benchmarks a Spikformer adapted from the public spikformer
CIFAR model (Models/spikformer_github.py:58-384): SPS patch embedding (four
conv3x3 + BN + LIF stages with two 3x3/2 max-pools and a relative position
conv), `depth` blocks of spiking self-attention (SSA: q/k/v Linear + BN +
LIF, attn = q @ k^T * scale, attn @ v, LIF, proj Linear + BN + LIF) and a
spiking MLP, then a token mean, LIF and a Linear head.  Its neurons are
spikingjelly LIFNodes (tau 2, hard reset to 0) switched to multi-step mode
(Benchmark/bench_4test.py:196); spikingjelly is not installed here, so the
network is restated with this package's multi-step LIFNode.

Activations: images [T, B, C, H, W]; tokens [T, B, N, C].
"""

from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn

from ..neuron import LIFNode


def _lif(v_threshold: float) -> LIFNode:
    return LIFNode(tau=2.0, v_threshold=v_threshold, v_reset=0.0, detach_reset=True, step_mode="m")


def _bn_tokens(bn: nn.Module, y: torch.Tensor) -> torch.Tensor:
    """BatchNorm1d over the channel axis of [TB, N, C] tokens."""
    return bn(y.transpose(-1, -2)).transpose(-1, -2)


class SpikingMLP(nn.Module):
    def __init__(self, dim: int, hidden_dim: int, v_threshold: float = 1.0):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden_dim)
        self.fc1_bn = nn.BatchNorm1d(hidden_dim)
        self.fc1_lif = _lif(v_threshold)
        self.fc2 = nn.Linear(hidden_dim, dim)
        self.fc2_bn = nn.BatchNorm1d(dim)
        self.fc2_lif = _lif(v_threshold)
        self.dim, self.hidden_dim = dim, hidden_dim

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        t, b, n, _ = x.shape
        y = _bn_tokens(self.fc1_bn, self.fc1(x.flatten(0, 1))).reshape(t, b, n, self.hidden_dim).contiguous()
        y = self.fc1_lif(y)
        y = _bn_tokens(self.fc2_bn, self.fc2(y.flatten(0, 1))).reshape(t, b, n, self.dim).contiguous()
        return self.fc2_lif(y)


class SSA(nn.Module):
    """Spiking self-attention (no softmax)."""

    def __init__(self, dim: int, num_heads: int, v_threshold: float = 1.0):
        super().__init__()
        if dim % num_heads != 0:
            raise ValueError(f"dim={dim} must be divisible by num_heads={num_heads}")
        self.dim, self.num_heads = dim, num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        for name in ("q", "k", "v"):
            setattr(self, name, nn.Linear(dim, dim))
            setattr(self, f"{name}_bn", nn.BatchNorm1d(dim))
            setattr(self, f"{name}_lif", _lif(v_threshold))
        self.attn_lif = _lif(v_threshold)
        self.proj = nn.Linear(dim, dim)
        self.proj_bn = nn.BatchNorm1d(dim)
        self.proj_lif = _lif(v_threshold)

    def _linear_bn_lif(self, x, linear, bn, lif):
        t, b, n, c = x.shape
        return lif(_bn_tokens(bn, linear(x.flatten(0, 1))).reshape(t, b, n, c).contiguous())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        t, b, n, c = x.shape
        heads = lambda z: z.reshape(t, b, n, self.num_heads, self.head_dim).permute(0, 1, 3, 2, 4).contiguous()  # noqa: E731
        q = heads(self._linear_bn_lif(x, self.q, self.q_bn, self.q_lif))
        k = heads(self._linear_bn_lif(x, self.k, self.k_bn, self.k_lif))
        v = heads(self._linear_bn_lif(x, self.v, self.v_bn, self.v_lif))
        attn = torch.matmul(q, k.transpose(-2, -1).contiguous()) * self.scale
        y = torch.matmul(attn, v)
        y = self.attn_lif(y.transpose(2, 3).reshape(t, b, n, c).contiguous())
        y = _bn_tokens(self.proj_bn, self.proj(y.flatten(0, 1))).reshape(t, b, n, c).contiguous()
        return self.proj_lif(y)


class SpikformerBlock(nn.Module):
    def __init__(self, dim: int, num_heads: int, mlp_ratio: float = 4.0, v_threshold: float = 1.0):
        super().__init__()
        self.attn = SSA(dim, num_heads, v_threshold)
        self.mlp = SpikingMLP(dim, int(dim * mlp_ratio), v_threshold)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(x)
        return x + self.mlp(x)


class SPS(nn.Module):
    """Spiking patch splitting: [T, B, C_in, H, W] -> tokens [T, B, H/4 * W/4, D]."""

    def __init__(self, in_channels: int, embed_dim: int, v_threshold: float = 1.0):
        super().__init__()
        chans = [in_channels, embed_dim // 8, embed_dim // 4, embed_dim // 2, embed_dim]
        for i in range(4):
            setattr(self, f"conv{i}", nn.Conv2d(chans[i], chans[i + 1], 3, 1, 1, bias=False))
            setattr(self, f"bn{i}", nn.BatchNorm2d(chans[i + 1]))
            setattr(self, f"lif{i}", _lif(v_threshold))
        self.pool2 = nn.MaxPool2d(3, 2, 1)
        self.pool3 = nn.MaxPool2d(3, 2, 1)
        self.rpe_conv = nn.Conv2d(embed_dim, embed_dim, 3, 1, 1, bias=False)
        self.rpe_bn = nn.BatchNorm2d(embed_dim)
        self.rpe_lif = _lif(v_threshold)

    @staticmethod
    def _conv_bn_lif(y, conv, bn, lif, t, b):
        y = bn(conv(y))
        y = lif(y.reshape(t, b, *y.shape[1:]).contiguous())
        return y.flatten(0, 1)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        t, b = x.shape[0], x.shape[1]
        y = x.flatten(0, 1).contiguous()
        y = self._conv_bn_lif(y, self.conv0, self.bn0, self.lif0, t, b)
        y = self._conv_bn_lif(y, self.conv1, self.bn1, self.lif1, t, b)
        y = self._conv_bn_lif(y, self.conv2, self.bn2, self.lif2, t, b)
        y = self.pool2(y)
        y = self._conv_bn_lif(y, self.conv3, self.bn3, self.lif3, t, b)
        y = self.pool3(y)
        feat = y.reshape(t, b, *y.shape[1:]).contiguous()
        r = self.rpe_bn(self.rpe_conv(y))
        r = self.rpe_lif(r.reshape(t, b, *r.shape[1:]).contiguous())
        y = r + feat
        return y.flatten(-2).transpose(-1, -2).contiguous()


class Spikformer(nn.Module):
    def __init__(self, img_size: Tuple[int, int] = (32, 32), in_channels: int = 3, num_classes: int = 10,
                 embed_dim: int = 384, num_heads: int = 12, mlp_ratio: float = 4.0, depth: int = 4, T: int = 4,
                 v_threshold: float = 1.0):
        super().__init__()
        self.img_size = tuple(img_size)
        self.T = int(T)
        self.num_classes = int(num_classes)
        self.patch_embed = SPS(in_channels, embed_dim, v_threshold)
        self.blocks = nn.ModuleList(SpikformerBlock(embed_dim, num_heads, mlp_ratio, v_threshold)
                                    for _ in range(depth))
        self.pre_head_lif = _lif(v_threshold)
        self.head = nn.Linear(embed_dim, num_classes) if num_classes > 0 else nn.Identity()
        for m in self.modules():
            if isinstance(m, nn.Linear):
                nn.init.trunc_normal_(m.weight, std=0.02)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
            elif isinstance(m, (nn.BatchNorm1d, nn.BatchNorm2d)):
                nn.init.ones_(m.weight)
                nn.init.zeros_(m.bias)

    def forward_features(self, x: torch.Tensor) -> torch.Tensor:
        y = self.patch_embed(x)
        for blk in self.blocks:
            y = blk(y)
        return y.mean(dim=2)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """[B, C, H, W] (repeated over T) or [T, B, C, H, W] -> logits [T, B, classes]."""
        if x.dim() == 4:
            x = x.unsqueeze(0).repeat(self.T, 1, 1, 1, 1)
        elif x.dim() != 5:
            raise ValueError(f"Expected 4D or 5D input, got shape={tuple(x.shape)}")
        y = self.pre_head_lif(self.forward_features(x))
        return self.head(y)


def spikformer_cifar_tiny(num_classes: int = 10, T: int = 4, v_threshold: float = 1.0) -> Spikformer:
    return Spikformer((32, 32), 3, num_classes, 192, 3, 4.0, 4, T, v_threshold)


def spikformer_cifar_small(num_classes: int = 10, T: int = 4, v_threshold: float = 1.0) -> Spikformer:
    return Spikformer((32, 32), 3, num_classes, 256, 8, 4.0, 6, T, v_threshold)


def spikformer_cifar_4_384(num_classes: int = 10, T: int = 4, v_threshold: float = 1.0) -> Spikformer:
    """Spikformer-4-384 on 32x32 inputs: dim 384, 12 heads (the attention
    workload's width), 8x8 = 64 tokens after the patch embedding."""
    return Spikformer((32, 32), 3, num_classes, 384, 12, 4.0, 4, T, v_threshold)


MODEL_BUILDERS = {
    "spikformer_cifar_tiny": spikformer_cifar_tiny,
    "spikformer_cifar_small": spikformer_cifar_small,
    "spikformer_cifar_4_384": spikformer_cifar_4_384,
}
