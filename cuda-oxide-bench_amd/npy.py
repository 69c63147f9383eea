"""NPY fixture I/O with the semantics of the reference's native loader, and
the reference's on-disk fixture sets.

The reference's kernels replay inputs written by its Python oracles
(pytorch_reference*.py, gen_kda_inputs.py) as `.npy` files in one
`inputs/` directory; its C++ cells read them with a small NPY parser
(cuda-attn-gqa/attn_gqa.cu:55-111):
  * magic ``\\x93NUMPY``, then a version byte pair; version 1.x stores the
    header length as a little-endian u16, versions 2.x and 3.x as a u32;
  * the header is a Python dict literal; ``'descr'`` must be ``'<f2'`` or
    ``'<f4'`` (anything else is an error), ``'shape'`` is a tuple of ints;
  * the payload is exactly prod(shape) elements, little-endian, C order;
    a short payload is an error.
`read_npy` follows that contract and is strict where the native parser is
silent: a Fortran-order header is rejected instead of being read as C
order.  `write_npy` writes version-1.0 files that numpy and the native
parser both read.

Fixture sets follow the reference's file names
(analysis/wave15-attention-architecture/reference/README.md:27-36, 83-86;
pytorch_reference.py:138-146, pytorch_reference_mla.py:159-168,
pytorch_reference_gdn.py:215-228, gen_kda_inputs.py:40-60):
  gqa_<shape>_{q,k,v}_{f16,f32}.npy, gqa_<shape>_expected_f32.npy
  mla_<shape>_{q,k,v}_{f16,f32}.npy, mla_<shape>_expected_f32.npy
  gdn_<shape>_{q,k,v,alpha,beta}_{f16,f32}.npy, gdn_<shape>_S_in_f32.npy,
      gdn_<shape>_o_expected_f16.npy, gdn_<shape>_S_out_expected_f32.npy
  kda_<shape>_{q,k,v,g,beta}_{f16,f32}.npy, kda_<shape>_S_in_f32.npy,
      kda_<shape>_o_expected_f16.npy, kda_<shape>_S_out_expected_f32.npy
"""
from __future__ import annotations

import ast
import struct
from pathlib import Path

import numpy as np

MAGIC = b"\x93NUMPY"
_DTYPES = {"<f2": np.float16, "<f4": np.float32}


class NpyError(ValueError):
    """A file that does not satisfy the fixture contract."""


def read_npy(path: str | Path) -> np.ndarray:
    """Read one fixture file; raises NpyError naming the file and the problem."""
    path = Path(path)
    try:
        f = open(path, "rb")
    except OSError as e:
        raise NpyError(f"cannot open {path}: {e}") from e
    with f:
        if f.read(6) != MAGIC:
            raise NpyError(f"{path}: not an NPY file")
        ver = f.read(2)
        if len(ver) != 2:
            raise NpyError(f"{path}: truncated header")
        major = ver[0]
        if major == 1:
            raw = f.read(2)
            if len(raw) != 2:
                raise NpyError(f"{path}: truncated header")
            (hlen,) = struct.unpack("<H", raw)
        elif major in (2, 3):
            raw = f.read(4)
            if len(raw) != 4:
                raise NpyError(f"{path}: truncated header")
            (hlen,) = struct.unpack("<I", raw)
        else:
            raise NpyError(f"{path}: unsupported NPY version {major}.{ver[1]}")
        hdr_bytes = f.read(hlen)
        if len(hdr_bytes) != hlen:
            raise NpyError(f"{path}: truncated header")
        try:
            hdr = ast.literal_eval(hdr_bytes.decode("latin1" if major < 3 else "utf8").strip())
        except (ValueError, SyntaxError) as e:
            raise NpyError(f"{path}: unreadable header") from e
        if not isinstance(hdr, dict) or "descr" not in hdr or "shape" not in hdr:
            raise NpyError(f"{path}: header lacks descr or shape")
        descr = hdr["descr"]
        if descr not in _DTYPES:
            raise NpyError(f"{path}: unsupported dtype {descr}")
        if hdr.get("fortran_order", False):
            raise NpyError(f"{path}: Fortran-order arrays are not fixtures")
        shape = tuple(int(d) for d in hdr["shape"])
        if any(d < 0 for d in shape):
            raise NpyError(f"{path}: negative dimension in shape {shape}")
        dt = np.dtype(_DTYPES[descr])
        n = 1
        for d in shape:
            n *= d
        payload = f.read(n * dt.itemsize)
        if len(payload) != n * dt.itemsize:
            raise NpyError(f"{path}: short read ({len(payload)} of {n * dt.itemsize} bytes)")
    return np.frombuffer(payload, dtype=dt).reshape(shape).copy()


def write_npy(path: str | Path, arr: np.ndarray) -> Path:
    """Write a float16/float32 array as an NPY 1.0 file (C order, little endian)."""
    arr = np.asarray(arr)
    descr = {np.dtype(np.float16): "<f2", np.dtype(np.float32): "<f4"}.get(arr.dtype)
    if descr is None:
        raise NpyError(f"fixtures hold float16 or float32, not {arr.dtype}")
    shape = repr(tuple(int(d) for d in arr.shape))
    hdr = f"{{'descr': '{descr}', 'fortran_order': False, 'shape': {shape}, }}"
    # pad so that magic + version + length + header + newline is a multiple of 64
    total = len(MAGIC) + 2 + 2 + len(hdr) + 1
    hdr = hdr + " " * ((64 - total % 64) % 64) + "\n"
    if len(hdr) > 0xFFFF:
        raise NpyError("header too long for NPY 1.0")
    path = Path(path)
    with open(path, "wb") as f:
        f.write(MAGIC + bytes([1, 0]) + struct.pack("<H", len(hdr)) + hdr.encode("latin1"))
        f.write(np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<"), copy=False).tobytes())
    return path


# role -> file suffix, per fixture kind; the 16-bit inputs are what the
# reference kernels consume, the f32 ones are kept alongside.
FIXTURE_FILES: dict[str, dict[str, str]] = {
    "gqa": {"q": "q_f16", "k": "k_f16", "v": "v_f16", "expected": "expected_f32"},
    "mla": {"q": "q_f16", "k": "k_f16", "v": "v_f16", "expected": "expected_f32"},
    "gdn": {"q": "q_f16", "k": "k_f16", "v": "v_f16", "alpha": "alpha_f16", "beta": "beta_f16",
            "S_in": "S_in_f32", "o_expected": "o_expected_f16", "S_out_expected": "S_out_expected_f32"},
    "kda": {"q": "q_f16", "k": "k_f16", "v": "v_f16", "g": "g_f16", "beta": "beta_f16",
            "S_in": "S_in_f32", "o_expected": "o_expected_f16", "S_out_expected": "S_out_expected_f32"},
}


def fixture_path(inputs_dir: str | Path, kind: str, shape_name: str, suffix: str) -> Path:
    return Path(inputs_dir) / f"{kind}_{shape_name}_{suffix}.npy"


def load_fixture_set(inputs_dir: str | Path, kind: str, shape_name: str) -> dict[str, np.ndarray]:
    """All files of one fixture set, by role; raises NpyError listing every missing file."""
    if kind not in FIXTURE_FILES:
        raise NpyError(f"unknown fixture kind {kind!r} (known: {', '.join(FIXTURE_FILES)})")
    roles = FIXTURE_FILES[kind]
    paths = {role: fixture_path(inputs_dir, kind, shape_name, suf) for role, suf in roles.items()}
    missing = [str(p) for p in paths.values() if not p.is_file()]
    if missing:
        raise NpyError("missing fixture files: " + ", ".join(missing))
    return {role: read_npy(p) for role, p in paths.items()}


def save_fixture_set(inputs_dir: str | Path, kind: str, shape_name: str, arrays: dict[str, np.ndarray]) -> list[Path]:
    """Write a fixture set under the reference's names (the 16-bit roles as
    float16, the f32 roles as float32)."""
    roles = FIXTURE_FILES[kind]
    out = []
    Path(inputs_dir).mkdir(parents=True, exist_ok=True)
    for role, suf in roles.items():
        dt = np.float16 if suf.endswith("f16") else np.float32
        out.append(write_npy(fixture_path(inputs_dir, kind, shape_name, suf), np.asarray(arrays[role]).astype(dt)))
    return out
