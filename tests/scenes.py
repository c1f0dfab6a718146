"""Small seeded scenes shared by the parity tests (sizes the oracle finishes in
seconds)."""
import numpy as np

from nest_splat.scene import get_spec, make_scene

# name -> overrides of the benchmark specs (same layouts, smaller sizes)
SMALL = {
    "cfg1": {},
    "shell_small": dict(name="shell_small", P=20_000, W=256, H=192, log2T=15),
    "unbounded_small": dict(name="unbounded_small", P=60_000, W=320, H=216, log2T=16),
    "shells_small": dict(name="shells_small", P=40_000, W=240, H=136, log2T=16, n_cams=2),
    "rvq_small": dict(name="rvq_small", P=20_000, W=200, H=200, log2T=15, rvq_codebook=512),
    # other channel counts per level (the table-gradient scatter splits entries by F)
    "unbounded_f8": dict(name="unbounded_f8", P=30_000, W=256, H=160, L=8, F=8, log2T=14),
    "unbounded_f1": dict(name="unbounded_f1", P=30_000, W=256, H=160, L=16, F=1, log2T=15),
}

_cache = {}


def scene(name):
    if name not in _cache:
        base = {"cfg1": "cfg1", "shell_small": "cfg2", "unbounded_small": "cfg3", "shells_small": "cfg5",
                "rvq_small": "cfg4", "unbounded_f8": "cfg3", "unbounded_f1": "cfg3"}[name]
        _cache[name] = make_scene(get_spec(base, **SMALL[name]))
    return _cache[name]
