"""Minimal PLY reader/writer for splat point clouds (no plyfile dependency).

Reads the first element of a PLY file in binary_little_endian,
binary_big_endian or ascii format (scalar properties only, the case of the
splat files scene/gaussian_model.py:554-589 writes), and writes one element
as binary little endian, which is what plyfile's PlyData.write produces for
those files.
"""
from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import numpy as np

_TYPES = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}
_NAMES = {"i1": "char", "u1": "uchar", "i2": "short", "u2": "ushort", "i4": "int", "u4": "uint", "f4": "float",
          "f8": "double"}


def _header(f) -> Tuple[str, List[Tuple[str, int, List[Tuple[str, str]]]]]:
    """(format, [(element, count, [(property, numpy type)])]); leaves f at the
    first byte of the body."""
    if f.readline().strip() != b"ply":
        raise ValueError("not a PLY file")
    fmt, elements = None, []
    while True:
        line = f.readline()
        if not line:
            raise ValueError("PLY header without end_header")
        tok = line.decode("ascii").strip().split()
        if not tok or tok[0] in ("comment", "obj_info"):
            continue
        if tok[0] == "format":
            fmt = tok[1]
        elif tok[0] == "element":
            elements.append((tok[1], int(tok[2]), []))
        elif tok[0] == "property":
            if not elements:
                raise ValueError("PLY property before any element")
            if tok[1] == "list":
                raise ValueError("list properties are not supported")
            if tok[1] not in _TYPES:
                raise ValueError(f"unknown PLY property type {tok[1]}")
            elements[-1][2].append((tok[2], _TYPES[tok[1]]))
        elif tok[0] == "end_header":
            break
    if fmt is None or not elements:
        raise ValueError("PLY header without format or element")
    return fmt, elements


def read_ply(path: str) -> Tuple[str, Dict[str, np.ndarray]]:
    """(element name, {property: array}) of the file's first element."""
    with open(path, "rb") as f:
        fmt, elements = _header(f)
        elem, count, props = elements[0]
        if fmt in ("binary_little_endian", "binary_big_endian"):
            end = "<" if fmt == "binary_little_endian" else ">"
            dt = np.dtype([(n, end + t) for n, t in props])
            data = np.frombuffer(f.read(dt.itemsize * count), dtype=dt, count=count)
            return elem, {n: np.asarray(data[n]).astype(np.dtype(t).newbyteorder("=")) for n, t in props}
        if fmt == "ascii":
            rows = [f.readline().split() for _ in range(count)]
            arr = np.array(rows, dtype=np.float64).reshape(count, len(props))
            return elem, {n: arr[:, i].astype(t) for i, (n, t) in enumerate(props)}
        raise ValueError(f"unknown PLY format {fmt}")


def write_ply(path: str, columns: Sequence[Tuple[str, np.ndarray]], element: str = "vertex") -> None:
    """One element of scalar properties, binary little endian."""
    if not columns:
        raise ValueError("no columns")
    n = int(np.asarray(columns[0][1]).shape[0])
    dt = np.dtype([(name, "<" + np.asarray(a).dtype.str[1:]) for name, a in columns])
    rec = np.empty(n, dtype=dt)
    for name, a in columns:
        a = np.asarray(a)
        if a.shape != (n,):
            raise ValueError(f"column {name} has shape {a.shape}, expected ({n},)")
        rec[name] = a
    head = ["ply", "format binary_little_endian 1.0", f"element {element} {n}"]
    head += [f"property {_NAMES[np.asarray(a).dtype.str[1:]]} {name}" for name, a in columns]
    head.append("end_header")
    with open(path, "wb") as f:
        f.write(("\n".join(head) + "\n").encode("ascii"))
        f.write(rec.tobytes())
