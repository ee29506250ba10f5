""".npz weight ingress on the GPU: dmc_hip_vault_load_npz against the oracle
(oracle/npz.py, the restatement of dmc_vault_load_npz, jit.rs:29836-29941),
bit for bit, through the C ABI; then a GEMV on a weight that arrived this way."""
import numpy as np
import pytest

import npz_files as F
import oracle
from oracle import npz as O
from parity import check

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def root(tmp_path_factory):
    return tmp_path_factory.mktemp("npz_gpu")


def loaded_bytes(hip, c: F.Case) -> bytes:
    buf = hip.vault_load_npz(c.path, c.key, c.numel, c.elem_bytes, c.convert)
    try:
        return buf.download(np.uint8, (buf.nbytes,)).tobytes()
    finally:
        buf.free()


def test_small_archives_bit_exact(hip, root):
    cases = F.all_small(root) + [F.zip64_case(root)]
    for c in cases:
        want = O.vault_load_npz(c.path, c.key, c.numel, c.elem_bytes, c.convert)
        assert want is not None, c.name
        if c.expect is not None:
            assert want == c.expect, c.name
        got = loaded_bytes(hip, c)
        assert got[:len(want)] == want, c.name
        assert got[len(want):] == bytes(16), c.name  # the zero padding


def test_failures_return_no_region(hip, root):
    why = {"missing_file": "cannot open", "not_a_zip": "not a valid zip file", "missing_key": "not found",
           "bad_magic": "not a valid .npy", "too_short_for_magic": "not a valid .npy",
           "v2_header_cut_short": "inside its .npy header", "crc_mismatch": "invalid checksum"}
    for c in F.error_cases(root):
        assert O.vault_load_npz(c.path, c.key, c.numel, c.elem_bytes, c.convert) is None, c.name
        with pytest.raises(hip.HipError) as e:
            hip.vault_load_npz(c.path, c.key, c.numel, c.elem_bytes, c.convert)
        assert why[c.name] in str(e.value), (c.name, str(e.value))


def test_large_stored_and_deflated(hip, root):
    """A C2 down weight (117 MB, stored: the parallel reader) and a 29 MB
    deflated one, checked against numpy.load's bytes; a corrupted byte in the
    large stored entry is caught by the CRC check on the parallel path."""
    for c in F.large_cases(root):
        buf = hip.vault_load_npz(c.path, c.key, c.numel, c.elem_bytes, c.convert)
        try:
            got = buf.download(np.uint16, (c.numel,))
        finally:
            buf.free()
        assert got.tobytes() == c.expect, c.name
        if c.name == "large_stored_c2_down":
            blob = bytearray(c.path.read_bytes())
            blob[len(blob) // 2] ^= 1  # inside the array data
            bad = root / "c2_corrupt.npz"
            bad.write_bytes(bytes(blob))
            with pytest.raises(hip.HipError, match="invalid checksum"):
                hip.vault_load_npz(bad, c.key, c.numel, 2, 0)


def test_gemv_on_an_ingested_weight(hip, root):
    """The path end to end: a bf16 weight saved with np.savez, loaded into HBM
    by the ingress, multiplied by the row-dot kernel, checked against the
    reference's chain."""
    rng = np.random.default_rng(5)
    n, k = 1536, 4096
    w = F.bf16_bits(rng, n * k).reshape(n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    p = root / "layer.npz"
    np.savez(p, wq=w)
    dw = hip.vault_load_npz(p, "wq", n * k, 2, 0)
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer(4 * n) as dy:
        hip.gemv_rd(dx, dw, dy, 1, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (1, n))
    dw.free()
    check(y, oracle.matmul_bf16_t(x, w), what="ingested gemv")


def test_f16_upconvert_every_pattern(hip):
    h = np.arange(65536, dtype=np.uint16)
    want = np.array([O.f16_bits_to_f32_bits(int(v)) for v in h], np.uint32)
    with hip.DeviceBuffer.from_numpy(h) as src, hip.DeviceBuffer(4 * h.size) as dst:
        for n in (65536, 65531):  # vector path, and the one-element tail
            hip.f16_upconvert(src, dst, n)
            hip.synchronize()
            assert np.array_equal(dst.download(np.uint32, (n,)), want[:n])
