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


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_eval_sh_matches_the_oracle(oracle, deg):
    """renderer.eval_sh (utils/sh_utils.py:57-117) + 0.5, clamped at 0, is the
    preprocess's SH colour (CR/forward.cu:21-72), which the oracle restates and
    scipy's spherical harmonics pin."""
    from nest_splat.renderer import eval_sh
    from nest_splat.scene import get_spec, make_scene
    sc = make_scene(get_spec("cfg1", P=500, name="sh_eval"))
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    shs = np.random.default_rng(deg).normal(0, 0.6, (500, 16, 3)).astype(np.float32)
    campos = np.asarray(cam.camera_center, np.float32)
    ref, _ = oracle.sh_colors(pre, sc.means, campos, shs, deg)
    d = torch.from_numpy(sc.means) - torch.from_numpy(campos)
    mine = torch.clamp_min(eval_sh(deg, torch.from_numpy(shs).transpose(1, 2), d / d.norm(dim=1, keepdim=True)) + 0.5,
                           0.0).numpy()
    vis = pre["radii"] > 0
    assert vis.sum() > 100
    assert np.abs(mine[vis] - ref[vis]).max() < 2e-6
