"""Archives for the .npz ingress tests, written at test time from fixed seeds.

Each builder writes one file under a directory and returns a Case: the path,
the key, the request (numel, elem_bytes, convert) as the JIT would lower
`vault.load_npz[T, shape]` (jit.rs:12671-12681), and what is expected --
either bytes checked by independent means (numpy.load, the reference's own
known answer) or None where the reference returns 0.
"""
from __future__ import annotations

import dataclasses
import io
import pathlib
import struct
import zipfile

import numpy as np


@dataclasses.dataclass
class Case:
    name: str
    path: pathlib.Path
    key: str
    numel: int
    elem_bytes: int
    convert: int
    expect: bytes | None = None   # the loaded buffer where it is known independently


def npy_bytes(a: np.ndarray, version=(1, 0)) -> bytes:
    buf = io.BytesIO()
    np.lib.format.write_array(buf, a, version=version, allow_pickle=False)
    return buf.getvalue()


def write_zip(path: pathlib.Path, entries: dict[str, bytes], method=zipfile.ZIP_STORED) -> pathlib.Path:
    with zipfile.ZipFile(path, "w", compression=method) as zf:
        for name, data in entries.items():
            zf.writestr(name, data)
    return path


def reference_kat(d: pathlib.Path) -> Case:
    """The archive of the reference's test jit_vault_load_npz_f32
    (jit.rs:41150-41191): an .npy v1 entry "test_key.npy" in a stored zip,
    header "{'descr': '<f4', 'fortran_order': False, 'shape': (4,), }"
    space-padded so that 10 + len + 1 is a multiple of 64, then '\\n', then
    f32 [5, 6, 7, 8]; the program sums the load to 26."""
    header = "{'descr': '<f4', 'fortran_order': False, 'shape': (4,), }"
    while (10 + len(header) + 1) % 64 != 0:
        header += " "
    header += "\n"
    npy = b"\x93NUMPY" + bytes([1, 0]) + struct.pack("<H", len(header)) + header.encode()
    npy += struct.pack("<4f", 5.0, 6.0, 7.0, 8.0)
    p = write_zip(d / "kat.npz", {"test_key.npy": npy})
    return Case("reference_kat_f32", p, "test_key", 4, 4, 0, struct.pack("<4f", 5.0, 6.0, 7.0, 8.0))


def bf16_bits(rng, n, scale=0.02) -> np.ndarray:
    v = (rng.standard_normal(n) * scale).astype(np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def numpy_cases(d: pathlib.Path) -> list[Case]:
    """Arrays saved by np.savez / np.savez_compressed; the expected bytes are
    numpy.load's, an independent reader of the same format."""
    rng = np.random.default_rng(7)
    arrays = {
        "w_bf16": bf16_bits(rng, 3 * 1031).reshape(3, 1031),        # odd length, bf16 bits
        "f32": rng.standard_normal((5, 7)).astype(np.float32),
        "f64": rng.standard_normal(9),
        "i64": rng.integers(-2**40, 2**40, 6),
        "mask": rng.integers(0, 2, 11).astype(bool),
        "empty": np.zeros((0, 4), np.uint16),
    }
    req = {"w_bf16": (2, 0), "f32": (4, 0), "f64": (8, 0), "i64": (8, 0), "mask": (1, 0), "empty": (2, 0)}
    cases = []
    for compressed in (False, True):
        p = d / ("savez_c.npz" if compressed else "savez.npz")
        (np.savez_compressed if compressed else np.savez)(p, **arrays)
        with np.load(p, allow_pickle=False) as z:
            for k, (eb, cv) in req.items():
                a = z[k]
                cases.append(Case(f"{p.stem}:{k}", p, k, a.size, eb, cv, a.tobytes()))
    return cases


def version_cases(d: pathlib.Path) -> list[Case]:
    """.npy format versions 1.0, 2.0 (4-byte header length) and 3.0."""
    a = bf16_bits(np.random.default_rng(11), 777)
    out = []
    for ver in ((1, 0), (2, 0), (3, 0)):
        for method in (zipfile.ZIP_STORED, zipfile.ZIP_DEFLATED):
            p = write_zip(d / f"v{ver[0]}_{method}.npz", {"a.npy": npy_bytes(a, ver)}, method)
            out.append(Case(f"npy_v{ver[0]}_m{method}", p, "a", a.size, 2, 0, a.tobytes()))
    return out


def key_cases(d: pathlib.Path) -> list[Case]:
    """Entry named "{key}" without ".npy" (jit.rs:29873-29878), and both present."""
    a = np.arange(10, dtype=np.uint16)
    b = np.arange(100, 110, dtype=np.uint16)
    p1 = write_zip(d / "bare.npz", {"w": npy_bytes(a)})
    p2 = write_zip(d / "both.npz", {"w": npy_bytes(b), "w.npy": npy_bytes(a), "other.npy": npy_bytes(b)})
    return [Case("bare_key", p1, "w", 10, 2, 0, a.tobytes()),
            Case("npy_preferred_over_bare", p2, "w", 10, 2, 0, a.tobytes())]


def short_cases(d: pathlib.Path) -> list[Case]:
    """Requests longer than the entry's data (jit.rs:29908-29919): what the
    entry holds, then zeros."""
    a = np.arange(1, 21, dtype=np.uint16)
    p = write_zip(d / "short.npz", {"a.npy": npy_bytes(a)})
    raw = npy_bytes(a)
    hdr = raw[:len(raw) - a.nbytes]
    p3 = write_zip(d / "hdr_only.npz", {"a.npy": hdr})
    return [Case("short_raw", p, "a", 32, 2, 0, a.tobytes() + bytes(24)),
            Case("short_f16", p, "a", 25, 2, 2, None),
            Case("header_only", p3, "a", 8, 2, 0, bytes(16))]


def widen_cases(d: pathlib.Path) -> list[Case]:
    """convert 1 (bf16 -> f32) and 2 (f16 -> f32) over every 16-bit pattern."""
    allbits = np.arange(65536, dtype=np.uint16)
    p = write_zip(d / "all16.npz", {"h.npy": npy_bytes(allbits)}, zipfile.ZIP_DEFLATED)
    return [Case("widen_bf16_all", p, "h", 65536, 2, 1, (allbits.astype(np.uint32) << 16).tobytes()),
            Case("widen_f16_all", p, "h", 65536, 2, 2, None)]


def error_cases(d: pathlib.Path) -> list[Case]:
    """Where the reference returns 0."""
    a = np.arange(64, dtype=np.uint16)
    good = write_zip(d / "good.npz", {"a.npy": npy_bytes(a)})
    notzip = d / "notzip.npz"
    notzip.write_bytes(b"this is not a zip archive" * 10)
    badmagic = write_zip(d / "badmagic.npz", {"a.npy": b"\x93NUMPZ" + npy_bytes(a)[6:]})
    tiny = write_zip(d / "tiny.npz", {"a.npy": b"\x93NUMPY\x01"})
    v2short = write_zip(d / "v2short.npz", {"a.npy": b"\x93NUMPY\x02\x00\x10\x00"})
    # A stored entry with one data byte flipped: its CRC-32 no longer matches.
    corrupt = d / "corrupt.npz"
    blob = bytearray(good.read_bytes())
    i = blob.index(npy_bytes(a)) + len(npy_bytes(a)) - 3
    blob[i] ^= 0x40
    corrupt.write_bytes(bytes(blob))
    return [Case("missing_file", d / "nope.npz", "a", 64, 2, 0),
            Case("not_a_zip", notzip, "a", 64, 2, 0),
            Case("missing_key", good, "b", 64, 2, 0),
            Case("bad_magic", badmagic, "a", 64, 2, 0),
            Case("too_short_for_magic", tiny, "a", 64, 2, 0),
            Case("v2_header_cut_short", v2short, "a", 64, 2, 0),
            Case("crc_mismatch", corrupt, "a", 64, 2, 0)]


def zip64_case(d: pathlib.Path) -> Case:
    """More than 65,535 entries: the archive's counts live in the ZIP64
    end-of-central-directory record (the 16-bit field reads 0xffff)."""
    p = d / "many.npz"
    a = np.arange(33, dtype=np.uint16)
    with zipfile.ZipFile(p, "w", compression=zipfile.ZIP_STORED) as zf:
        for i in range(65540):
            zf.writestr(f"e{i}", b"")
        zf.writestr("last.npy", npy_bytes(a))
    return Case("zip64_many_entries", p, "last", 33, 2, 0, a.tobytes())


def large_cases(d: pathlib.Path, n_rows=4096, k=14336) -> list[Case]:
    """A C2-sized bf16 weight (117 MB) stored, read by the parallel path, and a
    deflated one of 24 MB."""
    rng = np.random.default_rng(0)
    w = bf16_bits(rng, n_rows * k).reshape(n_rows, k)
    p = d / "c2_down.npz"
    np.savez(p, w=w)
    w2 = w[:1024, :].copy()
    p2 = d / "deflated.npz"
    np.savez_compressed(p2, w=w2)
    return [Case("large_stored_c2_down", p, "w", w.size, 2, 0, w.tobytes()),
            Case("large_deflated", p2, "w", w2.size, 2, 0, w2.tobytes())]


def all_small(d: pathlib.Path) -> list[Case]:
    return ([reference_kat(d)] + numpy_cases(d) + version_cases(d) + key_cases(d) + short_cases(d)
            + widen_cases(d))
