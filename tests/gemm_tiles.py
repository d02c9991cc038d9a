"""The GEMM's tile choice, read from the library itself
(``w8a8_gemm_tile_config``, the function ``launch_t`` in csrc/gemm.hip
dispatches on), so each test names the configuration its shape exercises on
the MI355X's 256 CUs.  The query makes no device call, so it also answers on a
machine without a GPU."""
from __future__ import annotations



def wd_fits(m: int, n: int, cus: int = 256) -> bool:
    """The weights-direct rule: one round of 112 x 256 tiles fills at least
    85% of the CUs, with at least 85% of the tile rows in use."""
    a = 7
    mb, nb = -(-m // 16), -(-n // 16)
    tm = -(-mb // a)
    tiles = tm * -(-nb // 16)
    return mb > 4 and tiles <= cus and 100 * tiles >= 85 * cus and 100 * mb >= 85 * tm * a


def narrow_fits(m: int, n: int, rows: int, cus: int = 256) -> bool:
    """The narrow-tile rule: one round of (16 rows) x 96 tiles, at least four
    tile rows, fills at least 80% of the CUs with at least 85% of the tile
    rows in use."""
    mb, nb = -(-m // 16), -(-n // 16)
    tm = -(-mb // rows)
    tiles = tm * -(-nb // 6)
    return mb > 4 and tm >= 4 and tiles <= cus and 100 * tiles >= 80 * cus and \
        100 * mb >= 85 * tm * rows


def gemm_config(m: int, n: int, cus: int = 256) -> str:
    from nanopointllm_amd import _lib

    code = _lib.load().w8a8_gemm_tile_config(m, n, cus)
    if code < 0:
        raise ValueError(f"no GEMM tile for {m} x {n}")
    return _lib.GEMM_TILE_NAMES[code]
