"""``turboquant.hadamard`` of the reference's module layout
(turboquant/hadamard.py): the normalised Walsh-Hadamard transform and the
sign-randomised rotation, from ``turboquant_amd.algorithm``."""
from .algorithm import RandomHadamardRotation, fwht, next_power_of_2

__all__ = ["fwht", "RandomHadamardRotation", "next_power_of_2"]
