"""On-disk formats of a trained scene: the splat PLY of scene/gaussian_model.py
(construct_list_of_attributes :533-552, save_ply :554-589, load_ply :597-686)
and the INGP checkpoint ngp_<iter>.pth (hash_encoder/modules.py:740-755).

PLY columns are the raw, pre-activation parameters: x y z, nx ny nz (zeros),
f_dc_0..2, f_rest_0.. (the SH rest coefficients channel-major: f_rest_{c*K+k}
is coefficient k+1 of channel c), opacity (logit), scale_0..1 (log),
rot_0..3 (unnormalised quaternion, w first), then gf_* (per-splat features)
and shape (beta kernel) when present.  The activations are
exp / normalise / sigmoid (scene/gaussian_model.py:26-41).  load_ply sets
the appearance level of every splat to 6 (:663-665), and so does load_ply
here.

The checkpoint holds {'model_state_dict': INGP.state_dict()}.  The hash grid
is a GridEncoder (gridencoder/grid.py:98-145): 'hash_encoding.embeddings'
[offsets[L], F] and the buffer 'hash_encoding.offsets' [L+1].  The colour MLP
is a tiny-cuda-nn Network whose parameters are one flat blob
('mlp_rgb.params'); the blob layout is not documented in the reference and no
trained checkpoint is available to check it against, so tcnn_mlp_weights
states the layout it assumes (parity unpinned).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np
import torch

from .plyio import read_ply, write_ply

LOAD_AP_LEVEL = 6.0  # gaussian_model.py:663-665


def ply_attributes(sh_degree: int, gf_dim: int = 0, has_shape: bool = False):
    """construct_list_of_attributes (gaussian_model.py:533-552)."""
    k_rest = (sh_degree + 1) ** 2 - 1
    names = ["x", "y", "z", "nx", "ny", "nz"] + [f"f_dc_{i}" for i in range(3)]
    names += [f"f_rest_{i}" for i in range(3 * k_rest)] + ["opacity", "scale_0", "scale_1"]
    names += [f"rot_{i}" for i in range(4)] + [f"gf_{i}" for i in range(gf_dim)]
    if has_shape:
        names.append("shape")
    return names


@dataclass
class RawSplats:
    """Raw splat parameters as GaussianModel holds them."""
    xyz: np.ndarray             # [P,3]
    features_dc: np.ndarray     # [P,1,3]
    features_rest: np.ndarray   # [P,K-1,3]
    opacity: np.ndarray         # [P,1] logit
    scaling: np.ndarray         # [P,2] log
    rotation: np.ndarray        # [P,4] unnormalised (w,x,y,z)
    gaussian_features: Optional[np.ndarray] = None  # [P,G]
    shape: Optional[np.ndarray] = None              # [P,1]

    @property
    def sh_degree(self) -> int:
        return int(round(np.sqrt(self.features_rest.shape[1] + 1))) - 1

    def shs(self) -> np.ndarray:
        """get_features: [P, K, 3] (DC first)."""
        return np.concatenate([self.features_dc, self.features_rest], axis=1).astype(np.float32)

    def activated(self) -> Dict[str, np.ndarray]:
        """get_scaling / get_rotation / get_opacity (gaussian_model.py:231-280):
        exp, normalize (x / max(|x|, 1e-12), torch.nn.functional.normalize)
        and sigmoid, in float32."""
        rot = self.rotation.astype(np.float32)
        norm = np.maximum(np.sqrt((rot * rot).sum(axis=1, keepdims=True)), np.float32(1e-12))
        op = self.opacity.astype(np.float32).reshape(-1, 1)
        with np.errstate(over="ignore"):
            sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-op))
        return {"xyz": self.xyz.astype(np.float32), "scales": np.exp(self.scaling.astype(np.float32)),
                "rotations": (rot / norm).astype(np.float32), "opacity": sig.astype(np.float32),
                "ap_level": np.full((self.xyz.shape[0], 1), LOAD_AP_LEVEL, np.float32)}


def save_splats_ply(path: str, s: RawSplats) -> None:
    """save_ply (gaussian_model.py:554-589): every column float32."""
    P = s.xyz.shape[0]
    f_dc = np.transpose(s.features_dc, (0, 2, 1)).reshape(P, -1)
    f_rest = np.transpose(s.features_rest, (0, 2, 1)).reshape(P, -1)
    parts = [s.xyz, np.zeros_like(s.xyz), f_dc, f_rest, s.opacity, s.scaling, s.rotation]
    if s.gaussian_features is not None and s.gaussian_features.shape[1] > 0:
        parts.append(s.gaussian_features)
    if s.shape is not None:
        parts.append(s.shape)
    attrs = np.concatenate([np.asarray(p, np.float32).reshape(P, -1) for p in parts], axis=1)
    names = ply_attributes(s.sh_degree, 0 if s.gaussian_features is None else s.gaussian_features.shape[1],
                           s.shape is not None)
    assert attrs.shape[1] == len(names)
    write_ply(path, [(n, attrs[:, i]) for i, n in enumerate(names)])


def _numbered(cols: Dict[str, np.ndarray], prefix: str):
    names = sorted((n for n in cols if n.startswith(prefix)), key=lambda n: int(n.split("_")[-1]))
    return names


def load_splats_ply(path: str, max_sh_degree: int = 3) -> RawSplats:
    """load_ply (gaussian_model.py:597-686)."""
    _, c = read_ply(path)
    P = c["x"].shape[0]
    xyz = np.stack([c["x"], c["y"], c["z"]], axis=1).astype(np.float32)
    opacity = np.asarray(c["opacity"], np.float32)[:, None]
    dc = np.stack([c["f_dc_0"], c["f_dc_1"], c["f_dc_2"]], axis=1).astype(np.float32).reshape(P, 3, 1)
    rest_names = _numbered(c, "f_rest_")
    k_rest = (max_sh_degree + 1) ** 2 - 1
    if len(rest_names) != 3 * k_rest:
        raise ValueError(f"{len(rest_names)} f_rest columns, expected {3 * k_rest} for SH degree {max_sh_degree}")
    rest = np.stack([c[n] for n in rest_names], axis=1).astype(np.float32).reshape(P, 3, k_rest) if k_rest else \
        np.zeros((P, 3, 0), np.float32)
    scales = np.stack([c[n] for n in _numbered(c, "scale_")], axis=1).astype(np.float32)
    rots = np.stack([c[n] for n in _numbered(c, "rot")], axis=1).astype(np.float32)
    gf_names = _numbered(c, "gf_")
    gf = np.stack([c[n] for n in gf_names], axis=1).astype(np.float32) if gf_names else None
    shape = np.asarray(c["shape"], np.float32)[:, None] if "shape" in c else None
    return RawSplats(xyz, np.transpose(dc, (0, 2, 1)).copy(), np.transpose(rest, (0, 2, 1)).copy(), opacity,
                     scales, rots, gf, shape)


# ---------------------------------------------------------------------------
# INGP checkpoint
# ---------------------------------------------------------------------------

def _next_multiple(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def tcnn_mlp_weights(params: np.ndarray, n_in: int, n_neurons: int, n_hidden_layers: int, n_out: int):
    """Split a tiny-cuda-nn "MLP" parameter blob into per-layer matrices
    [out, in] (input width padded to a multiple of 16, output to 16).
    Assumed layout, not checked against tiny-cuda-nn (parity unpinned):
    first layer [n_neurons, in16], n_hidden_layers - 1 hidden layers
    [n_neurons, n_neurons], last layer [out16, n_neurons], each row-major,
    concatenated in that order."""
    in16, out16 = _next_multiple(n_in, 16), _next_multiple(n_out, 16)
    shapes = [(n_neurons, in16)] + [(n_neurons, n_neurons)] * (n_hidden_layers - 1) + [(out16, n_neurons)]
    need = sum(a * b for a, b in shapes)
    flat = np.asarray(params, np.float32).reshape(-1)
    if flat.size != need:
        raise ValueError(f"tcnn MLP blob has {flat.size} values, the assumed layout needs {need}")
    mats, o = [], 0
    for a, b in shapes:
        mats.append(flat[o:o + a * b].reshape(a, b))
        o += a * b
    mats[0] = mats[0][:, :n_in]
    mats[-1] = mats[-1][:n_out]
    return [np.ascontiguousarray(m) for m in mats]


@dataclass
class NgpCheckpoint:
    embeddings: np.ndarray      # [offsets[L], F]
    offsets: np.ndarray         # [L+1] int
    mlp_params: Optional[np.ndarray]
    state: Dict[str, torch.Tensor]


def load_ngp(path: str) -> NgpCheckpoint:
    """load_model (hash_encoder/modules.py:750-755) with a loader that runs
    no code from the file (torch.load weights_only=True)."""
    ckpt = torch.load(path, map_location="cpu", weights_only=True)
    sd = ckpt["model_state_dict"] if isinstance(ckpt, dict) and "model_state_dict" in ckpt else ckpt
    if "hash_encoding.embeddings" not in sd or "hash_encoding.offsets" not in sd:
        raise KeyError("checkpoint has no hash_encoding.embeddings / hash_encoding.offsets")
    emb = sd["hash_encoding.embeddings"].detach().float().numpy()
    offs = sd["hash_encoding.offsets"].detach().cpu().numpy().astype(np.int64)
    mlp = sd.get("mlp_rgb.params")
    return NgpCheckpoint(emb, offs, None if mlp is None else mlp.detach().float().numpy(), dict(sd))


def save_ngp(path: str, embeddings: np.ndarray, offsets: np.ndarray, mlp_params: Optional[np.ndarray] = None) -> None:
    """save_model's container: {'model_state_dict': {...}} with the
    GridEncoder keys (and the MLP blob when given)."""
    sd = {"hash_encoding.embeddings": torch.from_numpy(np.ascontiguousarray(embeddings, np.float32)),
          "hash_encoding.offsets": torch.from_numpy(np.asarray(offsets, np.int32))}
    if mlp_params is not None:
        sd["mlp_rgb.params"] = torch.from_numpy(np.ascontiguousarray(mlp_params, np.float32))
    torch.save({"model_state_dict": sd}, path)
