"""CPU restatement of the reference's .npz weight loader.

TEST INFRASTRUCTURE ONLY: the checker for dmc_hip_vault_load_npz and the CPU
leg of its measurement.  The product package (demonic_amd) never imports it.

It restates, in plain Python over the standard library's `zipfile`:
  * dmc_vault_load_npz (compiler/src/jit.rs:29836-29926): open the archive,
    take the entry "{key}.npy" if present, else "{key}" (29873-29878), read it
    whole (the zip reader checks the CRC-32), require the .npy magic and at
    least 10 bytes (29895-29898), read the header length as 2 bytes at offset
    8 for major version 1 and as 4 bytes otherwise (29899-29906; a version-2+
    entry shorter than 12 bytes gives no buffer), and copy numel * elem_bytes
    bytes from the end of the header -- fewer when the entry is short
    (29908-29919);
  * npz_fill (jit.rs:29928-29941): convert 0 copies bytes, 1 widens bf16
    (bits << 16), 2 widens f16 through f16_bits_to_f32 (jit.rs:29231-29257),
    len(src) // 2 elements;
  * and one choice of this build: the part of the buffer an entry does not
    fill is zero (the reference leaves it as the arena held it).

Returns the loaded buffer as bytes, or None where the reference returns 0.
"""
from __future__ import annotations

import struct
import zipfile

# Planted mistakes for the pin tests (tests/test_npz.py); 0 = none.
MUTATIONS = {"v1_long_header_len": 1, "no_bare_key": 2, "data_off_by_one": 3, "f16_subnormal_exp": 4}
_mutation = 0


def set_mutation(m: int) -> None:
    global _mutation
    _mutation = m


def f16_bits_to_f32_bits(h: int) -> int:
    """IEEE binary16 -> binary32 bit pattern, exact (jit.rs:29231-29257)."""
    sign = (h & 0x8000) << 16
    exp = (h >> 10) & 0x1F
    mant = h & 0x3FF
    if exp == 0:
        if mant == 0:
            return sign
        # normalize: shift the fraction until its leading 1 reaches bit 10
        shifts = 0
        while not (mant & 0x400):
            mant <<= 1
            shifts += 1
        e = 127 - 15 - (shifts - 1)
        if _mutation == MUTATIONS["f16_subnormal_exp"]:
            e += 1
        return sign | (e << 23) | ((mant & 0x3FF) << 13)
    if exp == 0x1F:
        return sign | 0x7F800000 | (mant << 13)
    return sign | ((exp - 15 + 127) << 23) | (mant << 13)


def npz_fill(src: bytes, convert: int) -> bytes:
    """jit.rs:29928-29941."""
    if convert == 0:
        return bytes(src)
    n = len(src) // 2
    hs = struct.unpack(f"<{n}H", src[: 2 * n])
    if convert == 1:
        return struct.pack(f"<{n}I", *[h << 16 for h in hs])
    return struct.pack(f"<{n}I", *[f16_bits_to_f32_bits(h) for h in hs])


def npy_data_offset(raw: bytes):
    """Offset of the array data in an .npy entry, or None (jit.rs:29895-29907)."""
    if len(raw) < 10 or raw[:6] != b"\x93NUMPY":
        return None
    major = raw[6]
    if major == 1 and _mutation != MUTATIONS["v1_long_header_len"]:
        off = 10 + struct.unpack_from("<H", raw, 8)[0]
    else:
        if len(raw) < 12:
            return None
        off = 12 + struct.unpack_from("<I", raw, 8)[0]
    if _mutation == MUTATIONS["data_off_by_one"]:
        off += 1
    return off


def entry_name(names, key: str):
    """The entry the reference reads for `key` (jit.rs:29873-29878), or None."""
    if key + ".npy" in names:
        return key + ".npy"
    if _mutation == MUTATIONS["no_bare_key"]:
        return None
    return key if key in names else None


def vault_load_npz(path, key: str, numel: int, elem_bytes: int, convert: int):
    """The buffer dmc_vault_load_npz returns (as bytes), or None."""
    try:
        zf = zipfile.ZipFile(path)
    except (OSError, zipfile.BadZipFile):
        return None
    with zf:
        name = entry_name(set(zf.namelist()), key)
        if name is None:
            return None
        try:
            raw = zf.read(name)  # checks the CRC-32
        except (zipfile.BadZipFile, OSError, EOFError, NotImplementedError):
            return None
    off = npy_data_offset(raw)
    if off is None:
        return None
    src_bytes = numel * elem_bytes
    total = src_bytes if convert == 0 else numel * 4
    data = raw[off: off + src_bytes]
    out = bytearray(total)
    filled = npz_fill(data, convert)
    out[: len(filled)] = filled
    return bytes(out)
