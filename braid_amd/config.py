"""GDN shape constants (braid/config.py:6-66, :88-106).

Field names follow HF config.json as the reference's GDNConfig does:
``n_heads`` = linear_num_value_heads, ``head_dim`` = linear_value_head_dim (HD),
``state_size`` = linear_key_head_dim (SS), ``n_groups`` = linear_num_key_heads.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class GDNConfig:
    n_heads: int
    head_dim: int
    state_size: int
    n_groups: int
    conv_kernel: int = 4
    n_gdn_layers: int = 30

    @property
    def heads_per_group(self) -> int:
        return self.n_heads // self.n_groups

    @property
    def inner_size(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def key_dim(self) -> int:
        return self.n_groups * self.state_size

    @property
    def conv_channels(self) -> int:
        """[ Q (G*SS) | K (G*SS) | V (H*HD) ], Q first (braid/config.py:34-44)."""
        return 2 * self.key_dim + self.inner_size

    @staticmethod
    def _align256(n: int) -> int:
        return (n + 255) & ~255

    @property
    def state_bytes_per_seq_per_layer(self) -> int:
        """fp32 state, 256-byte aligned (braid/config.py:50-52)."""
        return self._align256(self.n_heads * self.state_size * self.head_dim * 4)

    @property
    def conv_bytes_per_seq_per_layer(self) -> int:
        return self._align256(self.conv_channels * self.conv_kernel * 4)

    @property
    def recurrent_bytes_per_seq(self) -> int:
        return (self.state_bytes_per_seq_per_layer
                + self.conv_bytes_per_seq_per_layer) * self.n_gdn_layers

    @classmethod
    def qwen35_9b(cls) -> "GDNConfig":
        """Qwen3.5-9B (and 4B): 32 value heads, 16 key heads, 128x128, 24 GDN layers."""
        return cls(n_heads=32, head_dim=128, state_size=128, n_groups=16, n_gdn_layers=24)

    @classmethod
    def qwen36_35b_a3b(cls) -> "GDNConfig":
        return cls(n_heads=32, head_dim=128, state_size=128, n_groups=16)
