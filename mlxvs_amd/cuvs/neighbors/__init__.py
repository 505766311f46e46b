"""cuVS's ``cuvs.neighbors``: the brute-force index."""

from mlxvs_amd.cuvs.neighbors import brute_force

__all__ = ["brute_force"]
