"""Host logic of render()'s SH-rasterised modes, on the CPU: the INGP point
normalisation (hash_encoder/modules.py:697-725) against the oracle's
restatement of query_feature's (hashgrid.h), with and without the contraction
of the space outside the unit ball, and the coarse-to-fine level mask
(modules.py:574-585, :692-695)."""
import numpy as np
import pytest
import torch

from nest_splat.renderer import HashINGP, render


class _Identity:
    """A stand-in encoding that returns its [0, 1] inputs, so encode_3D's
    normalisation is what the test sees."""
    num_levels = 3
    level_dim = 1

    def __call__(self, x):
        return x


@pytest.mark.parametrize("contract,gr", [(False, (-1.5, 1.5)), (True, (-1.0, 1.0)), (True, (-3.0, 2.0))])
def test_encode_normalisation_matches_oracle(oracle, contract, gr):
    rng = np.random.default_rng(3)
    pts = (rng.standard_normal((400, 3)) * 2.5).astype(np.float32)
    pts[:5] = 0.0
    ingp = HashINGP(_Identity(), mlp=None, gridrange=gr, contract=contract)
    got = ingp.encode_3D(torch.from_numpy(pts)).numpy()
    g = oracle.make_grid(1, 1, 1.0, 16, np.array([0, 8], np.int64), np.zeros((8, 1), np.float32), gr, contract)
    ref = np.stack([oracle.grid_normalise(g, p)[0] for p in pts])
    assert np.abs(got - ref).max() < 1e-6
    if contract:
        assert got.min() >= 0 and got.max() <= 1  # the contraction maps every point into the grid


def test_level_mask_zeroes_inactive_levels():
    ingp = HashINGP(_Identity(), mlp=None, gridrange=(0.0, 1.0), active_levels=2)
    out = ingp(torch.full((4, 3), 0.25))
    assert torch.equal(out[:, :2], torch.full((4, 2), 0.25)) and not out[:, 2:].any()
    withx = ingp(torch.full((4, 3), 0.25), with_xyz=True)
    assert withx.shape == (4, 6)


def test_unknown_mode_is_an_error():
    with pytest.raises(ValueError):
        render(None, None, None, torch.zeros(3), mode="residual")
