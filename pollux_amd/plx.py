""".plx container I/O: the reference's packed-checkpoint format, byte for byte.

Layout (pack.py:77-104, writer pack.py:187-247, readers generate.py:76-136
and evaluate.py:83-138), all integers little-endian:

    HEADER       16 B   b"POLLUXH2", version byte 0x04, 7 zero bytes
    CONFIG       u32 length, compact UTF-8 JSON (separators "," ":"), zero
                 padded so the next field starts on a 64-byte boundary of
                 the file
    FINGERPRINT  16 x f32 (codebook_fingerprint(), castor.py:263-266)
    COUNT        u32 number of tensors
    TENSOR       u16 name length, UTF-8 name, u8 dtype id (0 uint8, 1 int8,
                 2 float16, 3 float32), u8 ndim, ndim x u32 shape,
                 u64 byte length, raw C-order bytes

Tensors of other dtypes are stored as float32 (the writer's fallback,
pack.py:239-241).  ``read_plx`` returns the payload dict the reference's
readers return (format "pollux_packed_v4"); with ``mmap_file=True`` the
tensors are zero-copy views of a read-only memory map, so ``load_plx`` moves
packed weights from the page cache straight to the device.
"""

from __future__ import annotations

import json
import mmap
import struct
import warnings
from pathlib import Path
from typing import Any

import numpy as np
import torch

from .castor import codebook_fingerprint

PLX_MAGIC = b"POLLUXH2"
PLX_VERSION = 0x04
PLX_FORMAT = "pollux_packed_v4"

_ID_OF_DTYPE = {torch.uint8: 0, torch.int8: 1, torch.float16: 2, torch.float32: 3}
_NUMPY_OF_ID = {0: np.dtype("uint8"), 1: np.dtype("int8"), 2: np.dtype("<f2"), 3: np.dtype("<f4")}


def _config_pad(config_len: int) -> int:
    return (64 - (16 + 4 + config_len) % 64) % 64


def encode_plx(cfg_dict: dict, state: dict[str, torch.Tensor], fingerprint: tuple[float, ...] | None = None) -> bytes:
    """The .plx bytes of (config, state); ``fingerprint`` defaults to the canonical codebook's."""
    parts = [PLX_MAGIC, struct.pack("<B7x", PLX_VERSION)]
    cfg = json.dumps(cfg_dict, separators=(",", ":")).encode("utf-8")
    parts += [struct.pack("<I", len(cfg)), cfg, b"\x00" * _config_pad(len(cfg))]
    fp = list(codebook_fingerprint() if fingerprint is None else fingerprint)[:16]
    fp += [0.0] * (16 - len(fp))
    parts += [struct.pack("<16f", *fp), struct.pack("<I", len(state))]
    for name, tensor in state.items():
        t = tensor.detach()
        if t.dtype not in _ID_OF_DTYPE:
            t = t.to(torch.float32)
        t = t.contiguous().cpu()
        dtype_id = _ID_OF_DTYPE[t.dtype]
        raw = t.numpy().astype(_NUMPY_OF_ID[dtype_id], copy=False).tobytes()
        name_b = name.encode("utf-8")
        shape = list(t.shape)
        parts += [
            struct.pack("<H", len(name_b)), name_b,
            struct.pack("<BB", dtype_id, len(shape)), struct.pack(f"<{len(shape)}I", *shape),
            struct.pack("<Q", len(raw)), raw,
        ]
    return b"".join(parts)


def write_plx(path: str | Path, cfg_dict: dict, state: dict[str, torch.Tensor]) -> None:
    """pack._write_plx (pack.py:187-247)."""
    with open(path, "wb") as f:
        f.write(encode_plx(cfg_dict, state))


class _Reader:
    def __init__(self, buf, origin: str):
        self.buf, self.pos, self.origin = buf, 0, origin

    def take(self, n: int):
        if self.pos + n > len(self.buf):
            raise ValueError(f"{self.origin}: truncated .plx file (need {n} bytes at offset {self.pos})")
        view = self.buf[self.pos : self.pos + n]
        self.pos += n
        return view

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))


def decode_plx(buf, origin: str = "<bytes>", copy: bool = True) -> dict[str, Any]:
    """Parse .plx bytes (any buffer) into the reference's payload dict.

    copy=False returns tensors that view ``buf`` (read-only; torch warns on
    non-writable buffers, which is why ``read_plx`` copies unless asked not to).
    """
    r = _Reader(memoryview(buf), origin)
    magic = bytes(r.take(8))
    if magic != PLX_MAGIC:
        raise ValueError(f"{origin!r} is not a .plx file (bad magic {magic!r}).")
    (version,) = r.unpack("<B7x")
    if version != PLX_VERSION:
        raise ValueError(f"Unsupported .plx version {version} (expected {PLX_VERSION}).")
    (config_len,) = r.unpack("<I")
    config = json.loads(bytes(r.take(config_len)).decode("utf-8"))
    r.take(_config_pad(config_len))
    fingerprint = r.unpack("<16f")
    (n_tensors,) = r.unpack("<I")
    state: dict[str, torch.Tensor] = {}
    for _ in range(n_tensors):
        (name_len,) = r.unpack("<H")
        name = bytes(r.take(name_len)).decode("utf-8")
        dtype_id, ndim = r.unpack("<BB")
        shape = list(r.unpack(f"<{ndim}I"))
        (data_len,) = r.unpack("<Q")
        raw = r.take(data_len)
        np_dtype = _NUMPY_OF_ID.get(dtype_id, np.dtype("<f4"))
        count = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if count * np_dtype.itemsize != data_len:
            raise ValueError(f"{origin}: tensor {name!r} holds {data_len} bytes, shape {shape} needs "
                             f"{count * np_dtype.itemsize}")
        arr = np.frombuffer(raw, dtype=np_dtype).reshape(shape)
        if copy:
            arr = arr.copy()
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)  # read-only views of a memory map
            state[name] = torch.from_numpy(arr)
    return {"format": PLX_FORMAT, "config": config, "codebook_fingerprint": fingerprint, "state_dict": state}


def read_plx(path: str | Path, *, mmap_file: bool = False) -> dict[str, Any]:
    """generate._read_plx (generate.py:76-136).

    mmap_file=True maps the file read-only and returns zero-copy tensors
    (keep the payload alive while they are used).
    """
    path = str(path)
    if not mmap_file:
        with open(path, "rb") as f:
            return decode_plx(f.read(), path)
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    payload = decode_plx(mm, path, copy=False)
    payload["_mmap"] = mm
    return payload


def check_fingerprint(payload: dict[str, Any]) -> None:
    """The codebook check of PolluxModel.from_packed_checkpoint (pollux.py:714-724)."""
    if payload.get("format") != PLX_FORMAT:
        raise ValueError(f"Unsupported packed format: {payload.get('format')!r}")
    fp = payload.get("codebook_fingerprint")
    if fp is not None and tuple(fp) != codebook_fingerprint():
        raise ValueError(
            "H24 codebook fingerprint mismatch: packed checkpoint was built with a "
            "different kissing-point table than the current runtime."
        )


def load_plx(path: str | Path, device: torch.device | str) -> dict[str, Any]:
    """read_plx + check_fingerprint + the dtype normalisation of from_packed_checkpoint
    (pollux.py:729-740), with every tensor copied to ``device`` straight from the memory map
    (the map itself is released once the last view is gone)."""
    payload = read_plx(path, mmap_file=True)
    check_fingerprint(payload)
    out: dict[str, torch.Tensor] = {}
    for key, t in payload["state_dict"].items():
        if key.endswith(".packed_weights"):
            t = t.to(device=device, dtype=torch.uint8, copy=True)
        elif key.endswith(".weight_int8"):
            t = t.to(device=device, dtype=torch.int8, copy=True)
        elif key.endswith(".sigma_rows") or key.endswith(".mu_rows"):
            t = t.to(device=device, dtype=torch.float16, copy=True)
        elif t.is_floating_point():
            t = t.to(device=device, dtype=torch.float32, copy=True)
        else:
            t = t.to(device=device, copy=True)
        out[key] = t
    payload["state_dict"] = out
    del payload["_mmap"]
    return payload
