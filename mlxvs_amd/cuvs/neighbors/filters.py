"""cuVS's ``cuvs.neighbors.filters``: which rows a search may return.

The names, the two layouts and the bool-mask packing are cuVS's, as the
reference's compatibility module keeps them (python/mlxvs/cuvs/neighbors/
filters.py:10-50): a bitset holds one bit per dataset row (bit ``i % 32``
of word ``i // 32``), a bitmap one bit per (query, row), row-major over
``n_queries * n_rows`` bits with no padding per query.  A set bit allows the
row.  ``brute_force.search`` applies them inside the fused select.
"""

from __future__ import annotations

import numpy as np

__all__ = ["Prefilter", "from_bitmap", "from_bitset", "no_filter"]

_KINDS = ("none", "bitset", "bitmap")


class Prefilter:
    """A filter of the rows: ``type`` (``"none"``, ``"bitset"`` or
    ``"bitmap"``), ``array`` (its uint32 words) and ``parent`` (what it was
    made from)."""

    def __init__(self, type="none", array=None, parent=None):
        if type not in _KINDS:
            raise ValueError(f"a prefilter is one of {_KINDS}, not {type!r}")
        self.type = type
        self.array = array
        self.parent = parent

    def __repr__(self):
        return f"Prefilter(type={self.type!r})"


def _as_words(mask) -> np.ndarray:
    """uint32 words of a bool mask (its flattened bits little-endian, padded
    to whole words) or of an integer array of words."""
    if hasattr(mask, "copy_to_host"):
        mask = mask.copy_to_host()
    a = np.asarray(mask)
    if a.dtype == np.bool_:
        packed = np.packbits(a.reshape(-1), bitorder="little")
        return np.pad(packed, (0, (-packed.size) % 4)).view(np.uint32)
    if not np.issubdtype(a.dtype, np.integer):
        raise ValueError(f"filter words are unsigned integers or a bool mask, not {a.dtype}")
    return a.reshape(-1).astype(np.uint32, copy=False)


def no_filter() -> Prefilter:
    """Every row."""
    return Prefilter()


def from_bitset(bitset) -> Prefilter:
    """One bit per dataset row: uint32 words, or a bool mask ``[n_rows]``."""
    return Prefilter("bitset", _as_words(bitset), bitset)


def from_bitmap(bitmap) -> Prefilter:
    """One bit per (query, row), row-major: uint32 words of
    ``n_queries * n_rows`` bits, or a bool mask ``[n_queries, n_rows]``."""
    return Prefilter("bitmap", _as_words(bitmap), bitmap)
