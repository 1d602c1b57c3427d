"""Initialisation and learning-rate helpers (moc/optim.py:4-21)."""
import math


def moc_fan_in_std(k: int, kernel_size: int) -> float:
    """Variance-preserving init std sqrt(K / (3 S)) of the mixed kernel."""
    return math.sqrt(k / (3.0 * kernel_size))


def match_lr_to_init_std(init_std: float, reference_std: float = 0.002,
                         reference_lr: float = 1e-3) -> float:
    """Learning rate scaled in proportion to the init std."""
    return reference_lr * (init_std / reference_std)


def match_weight_decay_to_lr(lr: float, reference_lr: float = 1e-3,
                             reference_weight_decay: float = 0.1) -> float:
    """Weight decay scaled inversely with the learning rate (same lr*wd)."""
    return reference_weight_decay * (reference_lr / lr)
