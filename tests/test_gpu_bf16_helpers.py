"""GPU parity of the device bf16 helpers against the oracle, bit for bit.

dmc_hip_bf16_upconvert, dmc_hip_f32_to_bf16 and dmc_hip_bf16_transpose_2d are
the device forms of the reference's dmc_bf16_upconvert, dmc_f32_to_bf16 and
dmc_bf16_transpose_2d (compiler/src/jit.rs:29760, 29783, 29801).  Each case
runs once on 16-byte-aligned regions (the vector kernels) and once at an odd
2- or 4-byte offset (the element kernels).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def on_device(hip, host, offset, out_nbytes, out_offset, launch):
    """Upload `host` at `offset` bytes into a region, run `launch(src_addr,
    dst_addr)`, return the output region's bytes from `out_offset`."""
    with hip.DeviceBuffer(offset + max(host.nbytes, 1)) as ds, \
            hip.DeviceBuffer(out_offset + max(out_nbytes, 1)) as dd:
        if host.nbytes:
            ds.upload(host, offset=offset)
        launch(ds.addr + offset, dd.addr + out_offset)
        hip.synchronize()
        return dd.download(np.uint8, (out_nbytes,), offset=out_offset)


@pytest.mark.parametrize("offset,out_offset", [(0, 0), (2, 4), (0, 4), (6, 0)])
def test_upconvert_every_bf16_pattern(hip, offset, out_offset):
    """All 65,536 bit patterns (NaN payloads, infinities, subnormals, signed
    zeros) plus ragged counts."""
    for n in (65536, 65535, 65529, 9, 8, 1):
        h = np.arange(65536, dtype=np.uint16)[-n:] if n % 2 else np.arange(n, dtype=np.uint16) * 7
        got = on_device(hip, h, offset, 4 * n, out_offset,
                        lambda s, d: hip.bf16_upconvert(s, d, n)).view(np.uint32)
        want = oracle.widen(h).view(np.uint32)
        assert np.array_equal(got, want), (n, offset, out_offset, np.flatnonzero(got != want)[:8])


@pytest.mark.parametrize("offset,out_offset", [(0, 0), (4, 2), (0, 6), (12, 0)])
def test_f32_to_bf16_truncates_every_class(hip, offset, out_offset):
    rng = np.random.default_rng(offset * 10 + out_offset)
    bits = rng.integers(0, 2**32, size=200003, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001,
                        0x00000001, 0x807FFFFF, 0x00800000, 0x3F800000, 0x3F80FFFF, 0xBF7FFFFF], np.uint32)
    bits[:special.size] = special
    for n in (bits.size, 200000, 15, 8, 1):
        f = bits[:n].view(np.float32)
        got = on_device(hip, f, offset, 2 * n, out_offset,
                        lambda s, d: hip.f32_to_bf16(s, d, n)).view(np.uint16)
        want = oracle.truncate(f)
        assert np.array_equal(got, want), (n, offset, out_offset, np.flatnonzero(got != want)[:8])


@pytest.mark.parametrize("m,n", [(1, 1), (1, 9), (7, 3), (8, 8), (64, 64), (72, 136), (136, 72), (63, 65),
                                 (4097, 11008), (4096, 14336), (14336, 4096), (2, 40000)])
@pytest.mark.parametrize("offset", [0, 2])
def test_transpose_2d(hip, m, n, offset):
    """dst [n, m] = src [m, n]^T: rows and columns multiples of 8 on aligned
    regions take the 16-byte tile kernel (with partial edge tiles at 72, 136),
    the rest the element kernel."""
    rng = np.random.default_rng(m * 31 + n)
    w = rng.integers(0, 2**16, size=(m, n), dtype=np.uint64).astype(np.uint16)
    got = on_device(hip, w, offset, 2 * m * n, offset,
                    lambda s, d: hip.bf16_transpose_2d(s, d, m, n)).view(np.uint16).reshape(n, m)
    want = oracle.transpose(w)
    assert np.array_equal(got, want), (m, n, offset)


def test_zero_counts_do_nothing(hip):
    with hip.DeviceBuffer(64) as b:
        b.upload(np.full(16, 0xAB, np.uint32))
        hip.bf16_upconvert(b, b.addr + 32, 0)
        hip.f32_to_bf16(b, b.addr + 32, 0)
        hip.bf16_transpose_2d(b, b.addr + 32, 0, 5)
        hip.bf16_transpose_2d(b, b.addr + 32, 5, 0)
        hip.synchronize()
        assert np.all(b.download(np.uint32, (16,)) == 0xAB)


def test_bad_arguments_are_refused(hip):
    with pytest.raises(Exception):
        hip.bf16_upconvert(0, 0, 5)
    with pytest.raises(Exception):
        hip.f32_to_bf16(0, 0, -1)
    with pytest.raises(Exception):
        hip.bf16_transpose_2d(0, 0, -1, 3)
