"""View-direction MLP decode: the rgb_decode side of INGP
(hash_encoder/modules.py:551-602).

NestMLP holds the bias-free weights of the reference's network
(n_input = C + 16 -> width -> width -> 3, ReLU hidden, sigmoid output) as
float32 parameters plus cached copies in the compute dtype, and runs them on
libnest_splat: MFMA (v_mfma_f32_16x16x16 f16/bf16) for float16/bfloat16, the
vector ALU for float32.  The SphericalHarmonics degree-4 view encoding and the
(d+1)/2 input mapping are fused into the kernel.
"""
from __future__ import annotations

import ctypes as ct
import math
from typing import Optional

import numpy as np
import torch
import torch.nn as nn

from . import _lib as L

_DT = {"f32": (L.DTYPE_F32, torch.float32), "f16": (L.DTYPE_F16, torch.float16), "bf16": (L.DTYPE_BF16, torch.bfloat16),
       torch.float32: (L.DTYPE_F32, torch.float32), torch.float16: (L.DTYPE_F16, torch.float16),
       torch.bfloat16: (L.DTYPE_BF16, torch.bfloat16)}


class NestMLP(nn.Module):
    def __init__(self, in_features: int, width: int = 64, dtype="f16", W1=None, W2=None, W3=None, seed: int = 0):
        super().__init__()
        self.in_features = int(in_features)
        self.width = int(width)
        self.code, self.torch_dtype = _DT[dtype]
        Din = self.in_features + 16
        if W1 is None:
            g = torch.Generator().manual_seed(seed)

            def xavier(o, i):
                a = math.sqrt(6.0 / (i + o))
                return (torch.rand((o, i), generator=g) * 2 - 1) * a
            W1, W2, W3 = xavier(width, Din), xavier(width, width), xavier(3, width)
        self.W1 = nn.Parameter(torch.as_tensor(np.asarray(W1), dtype=torch.float32).clone())
        self.W2 = nn.Parameter(torch.as_tensor(np.asarray(W2), dtype=torch.float32).clone())
        self.W3 = nn.Parameter(torch.as_tensor(np.asarray(W3), dtype=torch.float32).clone())
        assert self.W1.shape == (width, Din) and self.W2.shape == (width, width) and self.W3.shape == (3, width)
        self._cache = None

    def _weights(self):
        key = (self.W1.device, self.W1._version, self.W2._version, self.W3._version, self.torch_dtype)
        if self._cache is None or self._cache[0] != key:
            ws = tuple(w.detach().to(self.torch_dtype).contiguous() for w in (self.W1, self.W2, self.W3))
            self._cache = (key, ws)
        return self._cache[1]

    def _desc(self):
        w1, w2, w3 = self._weights()
        m = L.Mlp()
        m.struct_size = ct.sizeof(L.Mlp)
        m.in_features = self.in_features
        m.width = self.width
        m.dtype = self.code
        m.w1, m.w2, m.w3 = w1.data_ptr(), w2.data_ptr(), w3.data_ptr()
        return m, (w1, w2, w3)

    def decode(self, feat: torch.Tensor, feat_cstride: int, feat_nstride: int, N: int, out: torch.Tensor,
               out_ostride: int, out_nstride: int, dirs: Optional[torch.Tensor] = None, ray_matrix=None,
               img_width: int = 0, alpha: Optional[torch.Tensor] = None, bg=None) -> torch.Tensor:
        if feat.dtype != torch.float32 or out.dtype != torch.float32:
            raise TypeError("features and output are float32")
        m, keep = self._desc()
        Mc = None
        if ray_matrix is not None:
            Mc = (ct.c_float * 9)(*[float(v) for v in np.asarray(ray_matrix, dtype=np.float32).reshape(-1)])
        bgc = None
        if bg is not None:
            b = np.asarray(bg.detach().cpu().numpy() if isinstance(bg, torch.Tensor) else bg, dtype=np.float32).reshape(-1)
            bgc = (ct.c_float * 3)(float(b[0]), float(b[1]), float(b[2]))
        if dirs is not None:
            dirs = dirs.detach().to(torch.float32).contiguous()
        if alpha is not None:
            alpha = alpha.detach().contiguous()
        L.check(L.lib().nest_mlp_decode(ct.byref(m), L.ptr(feat), feat_cstride, feat_nstride, N, int(img_width),
                                        L.ptr(dirs), Mc, L.ptr(alpha), bgc, L.ptr(out), out_ostride, out_nstride,
                                        L.stream_ptr(feat.device)), "nest_mlp_decode")
        return out

    def rgb_decode(self, features: torch.Tensor, ray_unit: torch.Tensor) -> torch.Tensor:
        """INGP.rgb_decode(features [N, C], ray_unit [N, 3]) -> rgb [N, 3]
        (HE:596).  Any strides of ``features`` are honoured, so the
        channel-major view color.view(C, -1).permute(1, 0) costs no copy."""
        N, C = features.shape
        if C != self.in_features:
            raise ValueError(f"expected {self.in_features} feature channels, got {C}")
        out = torch.empty((N, 3), dtype=torch.float32, device=features.device)
        return self.decode(features.detach(), features.stride(1), features.stride(0), N, out, 1, 3, dirs=ray_unit)

    def decode_image(self, color: torch.Tensor, ray_matrix, alpha: Optional[torch.Tensor] = None, bg=None) -> torch.Tensor:
        """color [C, H, W] -> rgb [3, H, W] with per-pixel view directions from
        ``ray_matrix`` (camera.view_ray_matrix), the alpha > 0 mask and the
        background composition of gaussian_renderer/__init__.py:1013-1021."""
        C, H, W = color.shape
        out = torch.empty((3, H, W), dtype=torch.float32, device=color.device)
        a = None if alpha is None else alpha.reshape(-1)
        return self.decode(color, H * W, 1, H * W, out, H * W, 1, ray_matrix=ray_matrix, img_width=W, alpha=a, bg=bg)
