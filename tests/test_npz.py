""".npz weight ingress on the CPU: the oracle (oracle/npz.py, the restatement
of dmc_vault_load_npz, jit.rs:29836-29941) pinned against the reference's own
known answers, numpy's reader and the published formats; and the library's
archive parser (dmc_hip_npz_locate, no device) against Python's zipfile."""
import struct
import zipfile

import numpy as np
import pytest

import demonic_amd as d
import npz_files as F
from oracle import npz as O


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    root = tmp_path_factory.mktemp("npz")
    return {"small": F.all_small(root), "errors": F.error_cases(root), "zip64": F.zip64_case(root)}


def load(c: F.Case):
    return O.vault_load_npz(c.path, c.key, c.numel, c.elem_bytes, c.convert)


# ---- oracle pins ----------------------------------------------------------------

def test_reference_kat_f32(files):
    """jit.rs:41150-41191: the stored v1 entry loads f32 [5, 6, 7, 8], sum 26."""
    c = next(c for c in files["small"] if c.name == "reference_kat_f32")
    got = load(c)
    assert got == c.expect
    assert sum(struct.unpack("<4f", got)) == 26.0


def test_reference_kat_bool_raw_copy():
    """jit.rs:30180-30197: convert 0 passes numpy bool bytes through 1:1."""
    assert O.npz_fill(bytes([1, 0, 1, 1]), 0) == bytes([1, 0, 1, 1])


def test_oracle_matches_independent_readers(files):
    """numpy.load (savez, savez_compressed, every dtype the JIT loads), the
    .npy versions 1-3, bare keys, short entries and the bf16 widen."""
    checked = 0
    for c in files["small"]:
        if c.expect is None:
            continue
        assert load(c) == c.expect, c.name
        checked += 1
    assert checked >= 20


def test_oracle_f16_widen_every_pattern():
    """f16 -> f32 over all 65,536 patterns: numpy's conversion for every
    non-NaN value (subnormals included); NaNs by the closed form of IEEE
    binary16 -> binary32 (sign, all-ones exponent, payload << 13) and class."""
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([O.f16_bits_to_f32_bits(int(v)) for v in h], np.uint32)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(got[~nan], ref[~nan])
    hv = h[nan].astype(np.uint32)
    assert np.array_equal(got[nan], ((hv & 0x8000) << 16) | 0x7F800000 | ((hv & 0x3FF) << 13))
    assert np.all(np.isnan(got[nan].view(np.float32)))
    # a few by hand: 1.0, -2.0, the smallest subnormal 2^-24, the largest 65504, +inf
    for hb, fb in ((0x3C00, 0x3F800000), (0xC000, 0xC0000000), (0x0001, 0x33800000),
                   (0x7BFF, 0x477FE000), (0x7C00, 0x7F800000)):
        assert O.f16_bits_to_f32_bits(hb) == fb


def test_oracle_short_request_reads_what_the_entry_holds(files):
    c = next(c for c in files["small"] if c.name == "short_f16")
    got = load(c)
    assert len(got) == 25 * 4
    vals = np.frombuffer(got, np.float32)
    assert np.array_equal(vals[:20], np.arange(1, 21, dtype=np.uint16).view(np.float16).astype(np.float32))
    assert not np.any(np.frombuffer(got, np.uint32)[20:])


def test_oracle_errors_give_none(files):
    for c in files["errors"]:
        assert load(c) is None, c.name


def test_oracle_zip64_archive(files):
    c = files["zip64"]
    with open(c.path, "rb") as f:
        f.seek(-22, 2)
        eocd = f.read(22)
    assert eocd[:4] == b"PK\x05\x06" and struct.unpack_from("<H", eocd, 10)[0] == 0xFFFF
    assert load(c) == c.expect


@pytest.mark.parametrize("mutation", sorted(O.MUTATIONS))
def test_planted_oracle_mistakes_fail_the_pins(files, mutation):
    """Each planted mistake changes at least one pinned answer."""
    O.set_mutation(O.MUTATIONS[mutation])
    try:
        bad = [c.name for c in files["small"] if c.expect is not None and load(c) != c.expect]
        h = np.arange(65536, dtype=np.uint16)
        fin = ~np.isnan(h.view(np.float16))
        f16 = np.array([O.f16_bits_to_f32_bits(int(v)) for v in h[fin]], np.uint32)
        if not np.array_equal(f16, h[fin].view(np.float16).astype(np.float32).view(np.uint32)):
            bad.append("f16_widen")
    finally:
        O.set_mutation(0)
    assert bad, mutation


# ---- the library's archive parser, no device ---------------------------------------

def zip_truth(path, name):
    """Entry facts from Python's zipfile and the local header."""
    with zipfile.ZipFile(path) as zf:
        info = zf.getinfo(name)
        raw = zf.read(name)
    with open(path, "rb") as f:
        f.seek(info.header_offset)
        lh = f.read(30)
    n, x = struct.unpack_from("<HH", lh, 26)
    return info, info.header_offset + 30 + n + x, raw


def test_locate_matches_zipfile(files):
    seen = set()
    for c in files["small"] + [files["zip64"]]:
        if (c.path, c.key) in seen:
            continue
        seen.add((c.path, c.key))
        with zipfile.ZipFile(c.path) as zf:
            name = O.entry_name(set(zf.namelist()), c.key)
        info, pos, raw = zip_truth(c.path, name)
        got = d.npz_locate(c.path, c.key)
        assert got["bare"] == int(name == c.key), c.name
        assert got["method"] == info.compress_type, c.name
        assert got["compressed"] == info.compress_size, c.name
        assert got["uncompressed"] == info.file_size, c.name
        assert got["data_pos"] == pos, c.name
        assert got["crc"] == info.CRC, c.name
        assert got["npy_data_offset"] == O.npy_data_offset(raw), c.name
        assert got["npy_major"] == raw[6], c.name


def test_locate_errors_name_the_cause(files):
    why = {"missing_file": "cannot open", "not_a_zip": "not a valid zip file", "missing_key": "not found"}
    for c in files["errors"]:
        if c.name in why:
            with pytest.raises(d.HipError) as e:
                d.npz_locate(c.path, c.key)
            assert e.value.code == -5 and why[c.name] in str(e.value), c.name
    bad = {c.name: c for c in files["errors"]}
    assert d.npz_locate(bad["bad_magic"].path, "a")["npy_data_offset"] == -1
    assert d.npz_locate(bad["too_short_for_magic"].path, "a")["npy_data_offset"] == -1
    assert d.npz_locate(bad["v2_header_cut_short"].path, "a")["npy_data_offset"] == -2


def test_load_rejects_bad_requests_before_touching_a_device(files):
    c = files["small"][0]
    from demonic_amd import _lib
    lib = _lib.load()
    for numel, eb, cv in ((-1, 2, 0), (4, 0, 0), (4, 4, 1), (4, 2, 3), (4, 9, 0)):
        assert lib.dmc_hip_vault_load_npz(str(c.path).encode(), c.key.encode(), numel, eb, cv) == 0
        assert b"bad numel" in lib.dmc_hip_last_error()
    assert lib.dmc_hip_vault_load_npz(None, b"k", 1, 2, 0) == 0
