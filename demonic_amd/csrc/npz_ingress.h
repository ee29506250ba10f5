// npz_ingress.h -- reading one array of a NumPy .npz archive for
// dmc_hip_vault_load_npz, the device form of the reference's
// dmc_vault_load_npz (compiler/src/jit.rs:29836-29944).  Host code only.
//
// An .npz is a ZIP archive whose entries are .npy files.  The reference opens
// it with the `zip` crate (8.6.0, compiler/Cargo.lock:1988-1991), takes the
// entry "{key}.npy", else "{key}", reads the whole entry (the crate checks
// its CRC-32 at the end), skips the .npy header and copies the bytes that
// follow.  This module locates the entry from the archive's central directory
// (ZIP64 included), and streams its uncompressed bytes from the file --
// stored entries by positioned reads, deflated ones through zlib -- so a
// caller can move them to the device without holding the whole entry in host
// memory.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace dmc {

struct NpzEntry {
    std::string name;     // entry name in the archive
    bool bare = false;    // found as "{key}" (no ".npy" suffix)
    int method = 0;       // 0 stored, 8 deflate
    uint64_t csize = 0;   // compressed bytes
    uint64_t usize = 0;   // uncompressed bytes
    uint64_t data_pos = 0;  // file offset of the entry's (compressed) data
    uint32_t crc = 0;     // CRC-32 of the uncompressed bytes, from the central directory
};

// Locates `key` in the archive open on `fd`.  Returns 0, or a nonzero value
// with a message in `err` ("not a valid zip file ...", "key ... not found").
int npz_find_entry(int fd, const std::string &key, NpzEntry &e, std::string &err);

// Sequential reader of an entry's uncompressed bytes, updating the CRC-32 of
// what it produced.
class NpzStream {
  public:
    NpzStream(int fd, const NpzEntry &e);
    ~NpzStream();
    NpzStream(const NpzStream &) = delete;
    NpzStream &operator=(const NpzStream &) = delete;
    // Up to n bytes into dst; returns the count (0 at the end of the entry)
    // or -1 with a message in err.
    int64_t read(uint8_t *dst, size_t n, std::string &err);
    uint64_t produced() const { return out_; }
    uint32_t crc() const { return crc_; }

  private:
    int fd_;
    NpzEntry e_;
    uint64_t in_ = 0, out_ = 0;
    uint32_t crc_ = 0;
    bool zinit_ = false, zend_ = false;
    void *zs_ = nullptr;  // z_stream
    std::vector<uint8_t> ibuf_;
};

// Offset of the array data within an .npy entry whose first n bytes are p:
// magic "\x93NUMPY", major version at byte 6, header length as a 2-byte
// little-endian value at byte 8 when the major version is 1, else as a 4-byte
// one (jit.rs:29895-29906).  -1: fewer than 10 bytes or a wrong magic ("not a
// valid .npy file"); -2: a version-2+ header cut short before byte 12 (the
// reference returns 0 without a message).
int64_t npy_data_offset(const uint8_t *p, size_t n, int *major);

// CRC-32 of a byte range (zlib's), and of two ranges joined.
uint32_t npz_crc32(uint32_t crc, const uint8_t *p, size_t n);
uint32_t npz_crc32_combine(uint32_t a, uint32_t b, uint64_t len_b);

// Reads exactly n bytes at offset off; false on a short read or an error.
bool pread_exact(int fd, void *buf, size_t n, uint64_t off);

}  // namespace dmc
