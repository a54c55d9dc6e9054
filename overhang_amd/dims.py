"""GDN layer dimensions and the named shapes this build is tested and measured on."""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class GdnDims:
    """Gated DeltaNet layer dimensions (the ``linear_*`` fields of a Qwen3.5/3.6
    config.json, read by overhang engines/qwen.c:190-192, 196)."""

    kh: int            # linear_num_key_heads
    vh: int            # linear_num_value_heads
    kd: int            # linear_key_head_dim
    vd: int            # linear_value_head_dim
    K: int = 4         # linear_conv_kernel_dim
    hidden: int = 0    # hidden_size
    eps: float = 1e-6  # rms_norm_eps

    @property
    def key_dim(self) -> int:
        return self.kh * self.kd

    @property
    def val_dim(self) -> int:
        return self.vh * self.vd

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.val_dim

    @property
    def rep(self) -> int:
        return self.vh // self.kh

    @property
    def state_bytes(self) -> int:
        return 4 * self.vh * self.kd * self.vd


# The reference's tiny oracle model (oracle/qwen_tiny/config.json:26-30).
TINY = GdnDims(kh=2, vh=4, kd=16, vd=16, K=4, hidden=64)
# The benchmark's small correctness layer.
CFG1 = GdnDims(kh=2, vh=4, kd=32, vd=32, K=4, hidden=128)
# Qwen3.6-35B-A3B GDN layer.
Q35B = GdnDims(kh=16, vh=32, kd=128, vd=128, K=4, hidden=2048)
