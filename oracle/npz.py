"""The reference's .npz writer restated in Python (Matrix.mm:3748-4085, matrix.h:1237).

TEST INFRASTRUCTURE ONLY: the checker for matrix::save_as_npz / matrix::load_npz.  Only tests/
import this module; the product (matrix_amd/) never does.

save_as_npz(arrays) returns the bytes the reference writes for matrices holding these arrays:
  - npy_descr_for_dtype (Matrix.mm:3748-3790): the descr per dtype code; BFloat16 raises;
  - npy_shape_tuple_string (Matrix.mm:3795-3804): "(" + items joined by "," + ")", with a
    trailing "," for rank 1 and no spaces;
  - build_npy_blob (Matrix.mm:3816-3842): magic, version 1.0, u16 header length, the dict
    "{'descr': ..., 'fortran_order': False, 'shape': ..., }" padded with spaces and a final
    newline to a multiple of 64 bytes counted from the file start, then the data;
  - crc32 (Matrix.mm:3846-3856): reflected 0xEDB88320, bit by bit;
  - save_as_npz (Matrix.mm:3857-4053): entries arr_<i>.npy, local headers, central directory and
    end record with the field values listed there.
"""
from __future__ import annotations

import struct

import numpy as np

# dtype codes of matrix.h:35-52
F32, F16, U8, I32, I16, U32, U16, BOOL, I8, C64, BF16, I64, U64 = range(13)

DESCR = {F32: "<f4", F16: "<f2", I32: "<i4", U32: "<u4", I16: "<i2", U16: "<u2", U8: "|u1", BOOL: "|b1",
         I8: "|i1", I64: "<i8", U64: "<u8", C64: "<c8"}


def crc32(data: bytes) -> int:
    """CRC-32 as Matrix.mm:3846-3856 computes it: eight conditional xors per byte."""
    crc = 0xFFFFFFFF
    for b in data:
        crc ^= b
        for _ in range(8):
            crc = (crc >> 1) ^ (0xEDB88320 if crc & 1 else 0)
    return crc ^ 0xFFFFFFFF


def shape_tuple(shape) -> str:
    s = "("
    for i, v in enumerate(shape):
        s += str(int(v))
        if len(shape) == 1 or i + 1 < len(shape):
            s += ","
    return s + ")"


def npy_blob(code: int, shape, data: bytes) -> bytes:
    if code not in DESCR:
        raise ValueError("npy_descr_for_dtype: no numpy dtype for code %d" % code)
    header = "{'descr': '" + DESCR[code] + "', 'fortran_order': False, 'shape': " + shape_tuple(shape) + ", }"
    pad = (64 - (10 + len(header) + 1) % 64) % 64
    header = header + " " * pad + "\n"
    return b"\x93NUMPY" + bytes([1, 0]) + struct.pack("<H", len(header)) + header.encode("ascii") + data


def save_as_npz(entries) -> bytes:
    """entries: [(dtype code, shape, row-major element bytes)] -> the archive's bytes."""
    if len(entries) > 0xFFFF:
        raise ValueError("more than 65535 entries")
    out = bytearray()
    central = bytearray()
    for i, (code, shape, data) in enumerate(entries):
        name = ("arr_%d.npy" % i).encode("ascii")
        blob = npy_blob(code, shape, bytes(data))
        crc = crc32(blob)
        offset = len(out)
        out += struct.pack("<IHHHHHIIIHH", 0x04034B50, 20, 0, 0, 0, 0, crc, len(blob), len(blob), len(name), 0)
        out += name + blob
        central += struct.pack("<IHHHHHHIIIHHHHHII", 0x02014B50, 20, 20, 0, 0, 0, 0, crc, len(blob), len(blob),
                               len(name), 0, 0, 0, 0, 0, offset)
        central += name
    cd_offset = len(out)
    out += central
    out += struct.pack("<IHHHHIIH", 0x06054B50, 0, 0, len(entries), len(entries), len(central), cd_offset, 0)
    return bytes(out)
