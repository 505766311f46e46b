"""cuVS's ``cuvs.neighbors``: the brute-force index and its prefilters."""

from mlxvs_amd.cuvs.neighbors import brute_force, filters

__all__ = ["brute_force", "filters"]
