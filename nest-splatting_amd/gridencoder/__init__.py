"""Drop-in gridencoder package (forward pass) on libnest_splat."""
from .grid import GridEncoder, grid_encode_forward  # noqa: F401
