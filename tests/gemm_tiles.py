"""The GEMM's tile choice (csrc/gemm.hip, launch_t) restated for the tests,
on the MI355X's 256 CUs with two workgroup slots each, so that each test can
assert the configuration its shape exercises."""
from __future__ import annotations


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def gemm_config(m: int, n: int, cus: int = 256) -> str:
    mb, nb = _cdiv(m, 16), _cdiv(n, 16)
    slots, tiles_m = 2 * cus, _cdiv(mb, 8)
    big = tiles_m * _cdiv(nb, 8)
    if big <= slots:
        if big > cus:
            return "big"
        small = _cdiv(mb, 4) * _cdiv(nb, 4)
        if small <= cus and _cdiv(mb, 2) * _cdiv(nb, 2) <= 3 * cus:
            return "tiny-deep"
        return "small-deep" if small <= slots else "big-deep"
    if tiles_m * _cdiv(nb, 12) <= slots:
        return "w192"
    if tiles_m * _cdiv(nb, 14) <= slots:
        return "w224"
    wide = tiles_m * _cdiv(nb, 16)
    if slots < wide and wide * 100 < slots * 125:
        return "big"
    return "w256"
