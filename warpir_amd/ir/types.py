"""Tile type descriptors of the WarpIR tile IR.

Same public names, field order, defaults and ``str()`` forms as the
reference type system (``warpir/ir/types.py:8-87``), because the printer
output and the builder scripts depend on them.

Wave-64 interpretation used by the CDNA4 lowering (the reference leaves
the thread mapping to the harness):

* ``SharedTileType`` is one block-wide tile resident in LDS.
* ``RegTileType`` / ``ColVecType`` are *per-wavefront* slices: the
  block-level tile is split over ``block_rows // rows`` x
  ``block_cols // cols`` wavefronts of 64 lanes.  The reference's
  per-warp slices (``tests/gemm_baseline_v2.py:33``) read the same way
  with "warp" replaced by "wavefront".
* ``GlobalType`` is a 4-D row-major tensor ``[batch, depth, rows, cols]``
  in HBM; ``-1`` marks a dimension that is only known at launch time.
  Tile coordinates used with a global are in units of its
  ``sub_tile_type`` (the reference's TMA box, ``types.py:40-50``).
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Union


class GPUType(str, Enum):
    """Element types of the IR (``types.py:8-10``)."""

    bf16 = "bf16"
    fp32 = "fp32"
    # additive: 32-bit unsigned counters (the split-K per-tile arrival counts)
    u32 = "u32"


class TileLayout(str, Enum):
    """Element order inside a tile (``types.py:13-15``)."""

    row_major = "row_major"
    col_major = "col_major"


def _tile_str(kind: str, dtype: GPUType, rows: int, cols: int, layout: TileLayout) -> str:
    return f"{kind}<{dtype.value}, {rows}x{cols}, {layout.value}>"


@dataclass(frozen=True)
class SharedTileType:
    """A ``rows x cols`` tile held in LDS (``types.py:18-26``)."""

    data_type: GPUType
    rows: int
    cols: int
    layout: TileLayout = TileLayout.row_major

    def __str__(self) -> str:
        return _tile_str("shared_tile", self.data_type, self.rows, self.cols, self.layout)


@dataclass(frozen=True)
class RegTileType:
    """A per-wavefront register tile (``types.py:29-37``)."""

    data_type: GPUType
    rows: int
    cols: int
    layout: TileLayout = TileLayout.row_major

    def __str__(self) -> str:
        return _tile_str("reg_tile", self.data_type, self.rows, self.cols, self.layout)


@dataclass(frozen=True)
class GlobalType:
    """A 4-D row-major tensor in global memory (``types.py:40-50``)."""

    data_type: GPUType
    sub_tile_type: SharedTileType
    batch: int = -1
    depth: int = -1
    rows: int = -1
    cols: int = -1

    def __str__(self) -> str:
        dims = ", ".join(str(d) for d in (self.batch, self.depth, self.rows, self.cols))
        return f"global<{self.data_type.value}, {dims}>"


@dataclass(frozen=True)
class SharedBufferType:
    """A ring of ``count`` shared tiles; mutable, not an SSA value (``types.py:53-60``)."""

    tile_type: SharedTileType
    count: int

    def __str__(self) -> str:
        return f"shared_buffer<{self.tile_type}, count={self.count}>"


@dataclass(frozen=True)
class ColVecType:
    """A per-row register vector of a ``rows x cols`` register tile (``types.py:63-71``)."""

    data_type: GPUType
    rows: int
    cols: int

    def __str__(self) -> str:
        return f"col_vec<{self.data_type.value}, {self.rows}x{self.cols}>"


@dataclass(frozen=True)
class RowVecType:
    """*Additive.* A per-column register vector of a ``rows x cols`` register
    tile: one value per column, shared by all rows (e.g. the per-query
    log-sum-exp across a key-major score tile in attention backward)."""

    data_type: GPUType
    rows: int
    cols: int

    def __str__(self) -> str:
        return f"row_vec<{self.data_type.value}, {self.rows}x{self.cols}>"


@dataclass(frozen=True)
class ScalarType:
    """A named scalar type (``types.py:74-79``)."""

    name: str

    def __str__(self) -> str:
        return self.name


class IntType(ScalarType):
    """The 32-bit integer scalar type (``types.py:82-84``)."""

    def __init__(self) -> None:
        super().__init__("int")


TypeRef = Union[GlobalType, IntType, SharedTileType, RegTileType, SharedBufferType, ColVecType]
