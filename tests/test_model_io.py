"""On-disk formats (no GPU): the splat PLY of scene/gaussian_model.py and the
ngp_<iter>.pth container.  The reference holds no PLY or checkpoint files, so
the schema is pinned by its construct_list_of_attributes / save_ply /
load_ply text: column names and order, float32, binary little endian, the
channel-major f_rest layout, the activations, ap_level = 6 after a load, and
byte-exact round trips.  The tiny-cuda-nn MLP blob layout is unpinned."""
import os

import numpy as np
import pytest
import torch

from nest_splat import model_io as M
from nest_splat.plyio import read_ply, write_ply


def _raw(P=50, deg=3, gf=0, shape=False, seed=0):
    rng = np.random.default_rng(seed)
    K = (deg + 1) ** 2
    return M.RawSplats(rng.normal(size=(P, 3)).astype(np.float32), rng.normal(size=(P, 1, 3)).astype(np.float32),
                       rng.normal(size=(P, K - 1, 3)).astype(np.float32), rng.normal(size=(P, 1)).astype(np.float32),
                       rng.normal(-4, 0.5, (P, 2)).astype(np.float32), rng.normal(size=(P, 4)).astype(np.float32),
                       rng.normal(size=(P, gf)).astype(np.float32) if gf else None,
                       rng.uniform(0.5, 3, (P, 1)).astype(np.float32) if shape else None)


def test_attribute_list_matches_reference_order():
    names = M.ply_attributes(3)
    assert names[:9] == ["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1", "f_dc_2"]
    assert names[9:54] == [f"f_rest_{i}" for i in range(45)]
    assert names[54:] == ["opacity", "scale_0", "scale_1", "rot_0", "rot_1", "rot_2", "rot_3"]
    assert M.ply_attributes(0, gf_dim=2, has_shape=True)[-3:] == ["gf_0", "gf_1", "shape"]


@pytest.mark.parametrize("deg,gf,shape", [(3, 0, False), (0, 0, False), (2, 8, True)])
def test_ply_round_trip_and_byte_layout(tmp_path, deg, gf, shape):
    s = _raw(deg=deg, gf=gf, shape=shape)
    path = str(tmp_path / "point_cloud.ply")
    M.save_splats_ply(path, s)
    # independent parse of the bytes: ascii header, then packed little-endian float32 rows
    raw = open(path, "rb").read()
    head, body = raw.split(b"end_header\n", 1)
    lines = head.decode().splitlines()
    assert lines[0] == "ply" and lines[1] == "format binary_little_endian 1.0"
    assert lines[2] == f"element vertex {s.xyz.shape[0]}"
    props = [l.split() for l in lines[3:]]
    assert all(p[0] == "property" and p[1] == "float" for p in props)
    names = [p[2] for p in props]
    assert names == M.ply_attributes(deg, gf, shape)
    rows = np.frombuffer(body, dtype="<f4").reshape(s.xyz.shape[0], len(names))
    np.testing.assert_array_equal(rows[:, 0:3], s.xyz)
    assert not rows[:, 3:6].any()
    np.testing.assert_array_equal(rows[:, 6:9], s.features_dc[:, 0, :])
    K = (deg + 1) ** 2 - 1
    # f_rest_{c*K + k} = coefficient k+1 of channel c
    for c in range(3):
        for k in range(K):
            np.testing.assert_array_equal(rows[:, 9 + c * K + k], s.features_rest[:, k, c])
    back = M.load_splats_ply(path, max_sh_degree=deg)
    for f in ("xyz", "features_dc", "features_rest", "opacity", "scaling", "rotation", "gaussian_features", "shape"):
        a, b = getattr(s, f), getattr(back, f)
        if a is None:
            assert b is None
        else:
            np.testing.assert_array_equal(a, b, err_msg=f)
    assert back.sh_degree == deg
    shs = back.shs()
    assert shs.shape == (s.xyz.shape[0], (deg + 1) ** 2, 3)
    np.testing.assert_array_equal(shs[:, 0], s.features_dc[:, 0])


def test_load_rejects_wrong_sh_count(tmp_path):
    path = str(tmp_path / "p.ply")
    M.save_splats_ply(path, _raw(deg=1))
    with pytest.raises(ValueError):
        M.load_splats_ply(path, max_sh_degree=3)


def test_activations_and_load_ap_level():
    s = _raw(P=200)
    s.rotation[0] = 0.0
    a = s.activated()
    np.testing.assert_array_equal(a["scales"], np.exp(s.scaling))
    t = torch.from_numpy(s.opacity)
    np.testing.assert_allclose(a["opacity"], torch.sigmoid(t).numpy(), rtol=2e-7, atol=0)
    np.testing.assert_allclose(a["rotations"], torch.nn.functional.normalize(torch.from_numpy(s.rotation)).numpy(),
                               rtol=3e-7, atol=1e-30)
    assert not a["rotations"][0].any()  # zero quaternion -> zeros, as normalize
    assert (a["ap_level"] == 6.0).all()


def test_ply_reader_formats(tmp_path):
    """ascii and big-endian files with mixed property types and a second
    element read the same as the binary little-endian writer's output."""
    x = np.array([1.5, -2.0, 3.25], np.float32)
    k = np.array([7, 0, 255], np.uint8)
    asc = tmp_path / "a.ply"
    asc.write_text("ply\nformat ascii 1.0\ncomment made by hand\nelement vertex 3\nproperty float x\n"
                   "property uchar k\nelement face 0\nproperty list uchar int vertex_indices\nend_header\n"
                   "1.5 7\n-2 0\n3.25 255\n")
    with pytest.raises(ValueError):
        read_ply(str(asc))  # list properties are refused, even on a later element
    asc.write_text("ply\nformat ascii 1.0\ncomment made by hand\nelement vertex 3\nproperty float x\n"
                   "property uchar k\nend_header\n1.5 7\n-2 0\n3.25 255\n")
    name, cols = read_ply(str(asc))
    assert name == "vertex"
    np.testing.assert_array_equal(cols["x"], x)
    np.testing.assert_array_equal(cols["k"], k)
    be = tmp_path / "b.ply"
    rec = np.empty(3, dtype=[("x", ">f4"), ("k", "u1"), ("d", ">f8")])
    rec["x"], rec["k"], rec["d"] = x, k, x.astype(np.float64) * 2
    be.write_bytes(b"ply\nformat binary_big_endian 1.0\nelement vertex 3\nproperty float x\nproperty uchar k\n"
                   b"property double d\nend_header\n" + rec.tobytes())
    _, cols = read_ply(str(be))
    np.testing.assert_array_equal(cols["x"], x)
    np.testing.assert_array_equal(cols["d"], x.astype(np.float64) * 2)
    le = tmp_path / "c.ply"
    write_ply(str(le), [("x", x), ("k", k)])
    _, cols = read_ply(str(le))
    np.testing.assert_array_equal(cols["x"], x)
    np.testing.assert_array_equal(cols["k"], k)


def test_ngp_checkpoint_round_trip(tmp_path):
    rng = np.random.default_rng(2)
    offs = np.array([0, 4096, 12096, 20096], np.int32)
    emb = rng.normal(size=(offs[-1], 4)).astype(np.float32)
    n_in, N, hidden, n_out = 80, 64, 2, 3
    sizes = [(N, 80), (N, N), (16, N)]
    blob = rng.normal(size=sum(a * b for a, b in sizes)).astype(np.float32)
    path = str(tmp_path / "ngp_30000.pth")
    M.save_ngp(path, emb, offs, blob)
    ck = M.load_ngp(path)
    np.testing.assert_array_equal(ck.embeddings, emb)
    np.testing.assert_array_equal(ck.offsets, offs)
    W = M.tcnn_mlp_weights(ck.mlp_params, n_in, N, hidden, n_out)
    assert [w.shape for w in W] == [(N, 80), (N, N), (3, N)]
    np.testing.assert_array_equal(W[0], blob[:N * 80].reshape(N, 80))
    np.testing.assert_array_equal(W[2], blob[N * 80 + N * N:].reshape(16, N)[:3])
    with pytest.raises(ValueError):
        M.tcnn_mlp_weights(ck.mlp_params[:-1], n_in, N, hidden, n_out)
    # input width padded to 16: 70 inputs use an 80-wide first layer
    W70 = M.tcnn_mlp_weights(ck.mlp_params, 70, N, hidden, n_out)
    np.testing.assert_array_equal(W70[0], blob[:N * 80].reshape(N, 80)[:, :70])
