"""``turboquant.codebook`` of the reference's module layout
(turboquant/codebook.py): the Codebook class and the N(0, 1) Lloyd-Max
tables under the reference's names: ``_CENTROIDS_N01[b]`` the 2^b levels in
ascending order, ``_BOUNDARIES_N01[b]`` the midpoints between neighbours."""
from .algorithm import CENTROIDS_N01, Codebook

_CENTROIDS_N01 = {b: [-c for c in reversed(pos)] + list(pos) for b, pos in CENTROIDS_N01.items()}
_BOUNDARIES_N01 = {b: [(lv[i] + lv[i + 1]) / 2.0 for i in range(len(lv) - 1)]
                   for b, lv in _CENTROIDS_N01.items()}

__all__ = ["Codebook", "_CENTROIDS_N01", "_BOUNDARIES_N01"]
