"""Mixture-of-Convolutions on MI355X: drop-in for the reference ``moc`` package.

The forward, backward and decode paths run as hand-written gfx950 HIP kernels
in libmoc_hip.so, reached through a C ABI (include/moc_hip.h).
"""
from .api import MoC, MoCGroup, moc_hip, moc_triton, router_linear
from .optim import match_lr_to_init_std, match_weight_decay_to_lr, moc_fan_in_std

__all__ = [
    "MoC",
    "MoCGroup",
    "moc_triton",
    "moc_hip",
    "router_linear",
    "moc_fan_in_std",
    "match_lr_to_init_std",
    "match_weight_decay_to_lr",
]
