"""Drop-in gridencoder package on libnest_splat (forward, and backward for D = 3 float32 tables)."""
from .grid import GridEncoder, grid_encode, grid_encode_backward, grid_encode_forward  # noqa: F401
