"""The cuVS-compatible slice over the exact k-NN engine.

Only the brute-force module of reference python/mlxvs/cuvs (cuVS's
``cuvs.neighbors.brute_force``: build / search / save / load, and its index
file format) -- the index that is the exact k-NN path itself.
"""
