"""The TILE32 V layout helpers (kernels.tile_v / untile_v) on the CPU.

The layout is defined in include/kvq.h: in each 32-token tile, lane L = 16 g + c owns
bytes [32 L, 32 L + 32); its dword 2 p + k holds packed bytes (4 c + 2 k, 4 c + 2 k + 1)
of the tokens a = 0, 1 of k-slot pair p, token r = 16 (p // 2) + 4 g + 2 (p % 2) + a.
"""
import pytest
import torch

from llm_kvcache_quantization_amd.kernels import TILE_BYTES, tile_v, untile_v


def marked_rows(T):
    """rows[r, bi] = a unique byte per (r mod 32, bi mod 8) position pattern."""
    g = torch.Generator().manual_seed(T)
    return torch.randint(0, 256, (2, 3, T, 64), generator=g, dtype=torch.uint8)


@pytest.mark.parametrize("T", [1, 31, 32, 33, 100, 256])
def test_round_trip(T):
    rows = marked_rows(T)
    tiles = tile_v(rows)
    assert tiles.shape == (2, 3, (T + 31) // 32, TILE_BYTES)
    assert torch.equal(untile_v(tiles, T), rows)


def test_padding_is_zero():
    rows = torch.full((1, 1, 5, 64), 0xAB, dtype=torch.uint8)
    tiles = tile_v(rows)
    assert int((tiles != 0).sum()) == 5 * 64


@pytest.mark.parametrize("r,bi,offset", [
    (0, 0, 0),          # lane 0, dword 0, token a = 0, low byte
    (0, 1, 1),          # j = 1: the next byte of the same token
    (1, 0, 2),          # a = 1: the pair's second token fills bytes 2..3
    (0, 2, 4),          # k = 1: dword 1
    (2, 0, 8),          # p = 1 (tokens 2, 3): dword 2
    (16, 0, 16),        # p = 2 (second row block): dword 4
    (19, 3, 4 * 7 + 2 + 1),  # p = 3, k = 1, a = 1, j = 1: last byte of lane 0
    (0, 4, 32),         # c = 1: lane 1
    (4, 0, 16 * 32),    # g = 1: lane 16
    (31, 63, 2047),     # last byte of the tile
])
def test_known_positions(r, bi, offset):
    rows = torch.zeros(1, 1, 32, 64, dtype=torch.uint8)
    rows[0, 0, r, bi] = 7
    tiles = tile_v(rows)
    assert tiles[0, 0, 0, offset] == 7
    assert int(tiles.count_nonzero()) == 1


def test_lane_bytes_are_its_pv_operand():
    """Lane (g, c) of a tile holds exactly tokens {4g..4g+3, 16+4g..16+4g+3}, bytes
    4c..4c+3: the 8 tokens whose probabilities lane group g holds after QK."""
    T = 64
    tok = torch.arange(T).view(1, 1, T, 1).expand(1, 1, T, 64)
    byte = torch.arange(64).view(1, 1, 1, 64).expand(1, 1, T, 64)
    code = (tok % 32) * 4 + (byte % 4)  # distinct within a lane's column slice
    col = byte // 4
    tiles_code = tile_v(code.to(torch.uint8))
    tiles_col = tile_v(col.to(torch.uint8))
    for t in range(2):
        for L in (0, 5, 17, 63):
            g, c = L // 16, L % 16
            got = tiles_code[0, 0, t, 32 * L:32 * L + 32]
            toks = sorted({int(v) // 4 for v in got})
            assert toks == [4 * g + i for i in range(4)] + [16 + 4 * g + i for i in range(4)]
            assert torch.all(tiles_col[0, 0, t, 32 * L:32 * L + 32] == c)
