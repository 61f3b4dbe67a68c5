"""The decoder's MLP output map in the oracle (orc_mlp_map; DecoderLayer::apply_mlp_output_map,
src/decoder_layer.cpp:198-210) pinned by closed forms and an independent float64 restatement:
- an identity full map gives y back exactly;
- a zero right factor gives y back exactly (the low-rank form adds its correction to y);
- one-hot factors (left[a, 1] = 1, right[1, b] = 1, rank 2) add column a to column b and
  leave the other columns alone, which fixes the orientation of both factors;
- random full and low-rank maps agree with numpy float64 within bf16 rounding."""
import numpy as np
import pytest

from affine_cases import to16
from attn_cases import bf


def rows(rng, M, H):
    return to16(rng.normal(0, 1, (M, H)), 0)


def test_identity_full_map(orc):
    rng = np.random.default_rng(1)
    H = 256
    y = rows(rng, 4, H)
    eye = to16(np.eye(H), 0)
    assert np.array_equal(orc.mlp_map(y, full=eye), y)


def test_zero_right_factor(orc):
    rng = np.random.default_rng(2)
    H, R = 256, 32
    y = rows(rng, 3, H)
    left = to16(rng.normal(0, 1, (H, R)), 0)
    right = np.zeros((R, H), np.uint16)
    assert np.array_equal(orc.mlp_map(y, left=left, right=right), y)


def test_one_hot_factors_move_one_column(orc):
    rng = np.random.default_rng(3)
    H, R, a, b = 256, 2, 17, 200
    y = rows(rng, 4, H)
    left = np.zeros((H, R), np.uint16)
    right = np.zeros((R, H), np.uint16)
    left[a, 1] = to16(np.array([1.0]), 0)[0]
    right[1, b] = to16(np.array([1.0]), 0)[0]
    out = orc.mlp_map(y, left=left, right=right)
    want = y.copy()
    want[:, b] = orc.bf16((bf(y[:, b]) + bf(y[:, a])).astype(np.float32))
    assert np.array_equal(out, want)


@pytest.mark.parametrize("rank", [0, 64])
def test_random_maps_match_numpy(orc, rank):
    rng = np.random.default_rng(4 + rank)
    H, M = 512, 4
    y = rows(rng, M, H)
    if rank == 0:
        full = to16(rng.normal(0, 1 / np.sqrt(H), (H, H)), 0)
        got, want = orc.mlp_map(y, full=full), bf(y).astype(np.float64) @ bf(full)
    else:
        left = to16(rng.normal(0, 1 / np.sqrt(H), (H, rank)), 0)
        right = to16(rng.normal(0, 0.1 / np.sqrt(rank), (rank, H)), 0)
        yf = bf(y).astype(np.float64)
        got, want = orc.mlp_map(y, left=left, right=right), yf + (yf @ bf(left)) @ bf(right)
    g = bf(got).astype(np.float64)
    assert np.linalg.norm(g - want) <= 1e-2 * np.linalg.norm(want)
