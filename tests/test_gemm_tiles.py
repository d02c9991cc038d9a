"""The GEMM tile rule (the library's ``w8a8_gemm_tile_config`` query) on the
LLaMA-7B prefill shapes whose tile choices were measured on MI355X:
which configuration each shape takes on the MI355X's 256 CUs.  The GPU tests
run every configuration for exactness; this pins the shape-to-configuration
map, and the rule's invariants over a sweep of shapes."""
from __future__ import annotations

import pytest

from gemm_tiles import gemm_config, narrow_fits, wd_fits

QKV, O, GATEUP, DOWN = 12288, 4096, 22016, 4096


@pytest.mark.parametrize("m,n,cfg", [
    (560, QKV, "wd7x2"), (768, QKV, "w192"), (1024, QKV, "w192"), (2048, QKV, "w256"),
    (560, O, "t112x96"), (567, O, "t128x96"), (567, QKV, "big"), (768, O, "big-deep"),
    (1024, O, "big-deep"), (480, QKV, "wd7x2"), (500, O, "t112x96"), (560, DOWN, "t112x96"),
    (640, O, "t128x96"), (641, O, "big-deep"), (448, O, "small-deep"),
    (560, GATEUP, "w224"), (768, GATEUP, "big"), (1024, GATEUP, "w256"),
    (64, QKV, "tiny-deep"), (128, O, "mid"), (256, O, "mid"), (65, DOWN, "mid"),
    (100, 1000, "tiny-deep"), (160, 8192, "small-deep"), (128, 8192, "mid"),
    (256, QKV, "big-deep"), (384, GATEUP, "w192"), (8192, 8192, "w256sq"),
    (2048, GATEUP, "w256sq"), (2040, GATEUP, "w256sq"),
    (2050, GATEUP, "w256"), (4096, O, "w256"), (4096, QKV, "w256sq"),
])
def test_llama7b_prefill_tiles(m, n, cfg):
    assert gemm_config(m, n) == cfg


def test_every_config_fits_one_round_or_is_the_widest():
    """Within one round of 512 workgroup slots the rule never leaves a config
    that would also fit with more tiles; past it, only 128x256, 128x128, or
    256x256 from two full rounds of those with no extra row padding."""
    for m in range(65, 4097, 37):
        for n in (4096, 11008, 12288, 22016, 32000):
            cfg = gemm_config(m, n)
            assert (cfg == "wd7x2") == wd_fits(m, n), (m, n, cfg)
            if cfg == "wd7x2":
                continue
            narrow = ("t112x96" if narrow_fits(m, n, 7) else
                      "t128x96" if narrow_fits(m, n, 8) else None)
            assert (cfg == narrow) if narrow else cfg not in ("t112x96", "t128x96"), (m, n, cfg)
            if narrow:
                continue
            mb, nb = -(-m // 16), -(-n // 16)
            tm = -(-mb // 8)
            tiles = {"w192": tm * -(-nb // 12), "w224": tm * -(-nb // 14),
                     "w256": tm * -(-nb // 16), "big": tm * -(-nb // 8)}
            if cfg in ("w192", "w224"):
                assert tiles[cfg] <= 512 and tiles["big"] > 512
            if cfg == "w224":
                assert tiles["w192"] > 512
            if cfg == "w256sq":
                assert tiles["w256"] > 512 and -(-mb // 16) * -(-nb // 16) >= 512
                assert 2 * -(-mb // 16) == tm
    # 64x32 tiles only past 64 rows, within one round and on at least half the CUs.
    for m in range(17, 1025, 13):
        for n in (1000, 2048, 4096, 8192, 12288, 22016):
            mb, nb = -(-m // 16), -(-n // 16)
            mid = -(-mb // 4) * -(-nb // 2)
            fits = mb > 4 and 128 <= mid <= 512 and -(-mb // 8) * -(-nb // 8) <= 512
            if wd_fits(m, n) or narrow_fits(m, n, 7) or narrow_fits(m, n, 8):
                continue
            assert (gemm_config(m, n) == "mid") == fits, (m, n)


def test_query_rejects_empty_or_oversized_problems():
    from nanopointllm_amd import _lib

    lib = _lib.load()
    for m, n, cus in ((0, 64, 256), (64, 0, 256), (64, 64, 0), (-1, 64, 256),
                      (2 ** 31, 64, 256)):
        assert lib.w8a8_gemm_tile_config(m, n, cus) == -1
    # Largest accepted row count: the tile round-up still fits a signed int.
    assert lib.w8a8_gemm_tile_config(2 ** 31 - 1 - 256, 4096, 256) >= 0
