// npz_ingress.cpp -- ZIP/.npy reading behind dmc_hip_vault_load_npz (see
// npz_ingress.h).  Host code only; no HIP calls here.
//
// The archive layout follows the published ZIP format (PKWARE APPNOTE): the
// end-of-central-directory record (EOCD) near the end of the file, the ZIP64
// EOCD locator and record when a count, size or offset does not fit its
// 16/32-bit field, one central-directory header per entry (sizes, CRC-32,
// method, offset of the entry's local header; ZIP64 "extended information"
// extra field id 0x0001 for the large values), and a local header in front of
// each entry's data.  Methods 0 (stored) and 8 (raw deflate) are read; NumPy
// writes one or the other (np.savez / np.savez_compressed).
#include "npz_ingress.h"

#include <errno.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>
#include <zlib.h>

#include <algorithm>

namespace dmc {
namespace {

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) { return (uint32_t)rd16(p) | ((uint32_t)rd16(p + 2) << 16); }
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

constexpr uint32_t kSigEocd = 0x06054b50u, kSigZ64Loc = 0x07064b50u, kSigZ64Eocd = 0x06064b50u,
                   kSigCentral = 0x02014b50u, kSigLocal = 0x04034b50u;
constexpr size_t kEocdLen = 22, kZ64LocLen = 20, kZ64EocdLen = 56, kCentralLen = 46, kLocalLen = 30;

int bad(std::string &err, const std::string &msg) {
    err = msg;
    return 1;
}

}  // namespace

bool pread_exact(int fd, void *buf, size_t n, uint64_t off) {
    uint8_t *p = static_cast<uint8_t *>(buf);
    while (n > 0) {
        const ssize_t r = pread(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

// CRC-32 of the ZIP format (reflected polynomial 0xEDB88320, initial and
// final complement; the same value as zlib's crc32()) by table slicing, 16
// bytes per step (the slicing-by-N method of Kounavis and Berry): table t
// holds the CRC contribution of a byte followed by t zero bytes.  About 4x
// the throughput of zlib 1.2.11's four-table loop on these hosts, which
// otherwise bounds the parallel ingress.
namespace {
struct Crc16Tables {
    uint32_t t[16][256];
    Crc16Tables() {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int b = 0; b < 8; ++b) c = (c & 1) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
            t[0][i] = c;
        }
        for (int k = 1; k < 16; ++k)
            for (uint32_t i = 0; i < 256; ++i) t[k][i] = (t[k - 1][i] >> 8) ^ t[0][t[k - 1][i] & 0xff];
    }
};
const Crc16Tables &crc_tables() {
    static const Crc16Tables tables;
    return tables;
}
}  // namespace

uint32_t npz_crc32(uint32_t crc, const uint8_t *p, size_t n) {
    const auto &T = crc_tables().t;
    uint32_t c = ~crc;
    while (n >= 16) {
        uint32_t w[4];
        memcpy(w, p, 16);  // little-endian host
        w[0] ^= c;
        c = T[15][w[0] & 0xff] ^ T[14][(w[0] >> 8) & 0xff] ^ T[13][(w[0] >> 16) & 0xff] ^ T[12][w[0] >> 24] ^
            T[11][w[1] & 0xff] ^ T[10][(w[1] >> 8) & 0xff] ^ T[9][(w[1] >> 16) & 0xff] ^ T[8][w[1] >> 24] ^
            T[7][w[2] & 0xff] ^ T[6][(w[2] >> 8) & 0xff] ^ T[5][(w[2] >> 16) & 0xff] ^ T[4][w[2] >> 24] ^
            T[3][w[3] & 0xff] ^ T[2][(w[3] >> 8) & 0xff] ^ T[1][(w[3] >> 16) & 0xff] ^ T[0][w[3] >> 24];
        p += 16;
        n -= 16;
    }
    while (n--) c = (c >> 8) ^ T[0][(c ^ *p++) & 0xff];
    return ~c;
}

uint32_t npz_crc32_combine(uint32_t a, uint32_t b, uint64_t len_b) {
    return (uint32_t)crc32_combine(a, b, (z_off_t)len_b);
}

int npz_find_entry(int fd, const std::string &key, NpzEntry &e, std::string &err) {
    struct stat st;
    if (fstat(fd, &st) != 0) return bad(err, std::string("stat failed: ") + strerror(errno));
    const uint64_t fsize = (uint64_t)st.st_size;
    const std::string not_zip = "not a valid zip file";
    if (fsize < kEocdLen) return bad(err, not_zip + " (too short for an end-of-central-directory record)");

    // The EOCD is the last 22 bytes plus a comment of at most 65535 bytes.
    const uint64_t tail = std::min<uint64_t>(fsize, kEocdLen + 65535);
    std::vector<uint8_t> t(tail);
    if (!pread_exact(fd, t.data(), tail, fsize - tail)) return bad(err, not_zip + " (read failed)");
    int64_t at = -1;
    for (int64_t i = (int64_t)tail - (int64_t)kEocdLen; i >= 0; --i) {
        if (rd32(&t[i]) == kSigEocd && (uint64_t)i + kEocdLen + rd16(&t[i + 20]) <= tail) {
            at = i;
            break;
        }
    }
    if (at < 0) return bad(err, not_zip + " (no end-of-central-directory record)");
    const uint64_t eocd_pos = fsize - tail + (uint64_t)at;
    uint64_t entries = rd16(&t[at + 10]), cd_size = rd32(&t[at + 12]), cd_off = rd32(&t[at + 16]);
    if (entries == 0xffff || cd_size == 0xffffffffu || cd_off == 0xffffffffu) {
        uint8_t loc[kZ64LocLen], rec[kZ64EocdLen];
        if (eocd_pos < kZ64LocLen || !pread_exact(fd, loc, kZ64LocLen, eocd_pos - kZ64LocLen) ||
            rd32(loc) != kSigZ64Loc)
            return bad(err, not_zip + " (ZIP64 locator missing)");
        const uint64_t rec_pos = rd64(loc + 8);
        if (rec_pos + kZ64EocdLen > fsize || !pread_exact(fd, rec, kZ64EocdLen, rec_pos) ||
            rd32(rec) != kSigZ64Eocd)
            return bad(err, not_zip + " (ZIP64 end-of-central-directory record missing)");
        entries = rd64(rec + 32);
        cd_size = rd64(rec + 40);
        cd_off = rd64(rec + 48);
    }
    if (cd_off > fsize || cd_size > fsize - cd_off) return bad(err, not_zip + " (central directory out of range)");

    std::vector<uint8_t> cd(cd_size);
    if (cd_size && !pread_exact(fd, cd.data(), cd_size, cd_off)) return bad(err, not_zip + " (read failed)");
    const std::string want_npy = key + ".npy";
    bool have_npy = false, have_bare = false;
    NpzEntry npy, bare;
    uint64_t pos = 0;
    for (uint64_t i = 0; i < entries; ++i) {
        if (pos + kCentralLen > cd_size || rd32(&cd[pos]) != kSigCentral)
            return bad(err, not_zip + " (bad central directory header)");
        const uint8_t *h = &cd[pos];
        const uint16_t flags = rd16(h + 8), method = rd16(h + 10);
        const uint32_t crc = rd32(h + 16);
        uint64_t csize = rd32(h + 20), usize = rd32(h + 24), local = rd32(h + 42);
        const uint16_t nlen = rd16(h + 28), xlen = rd16(h + 30), clen = rd16(h + 32);
        if (pos + kCentralLen + nlen + xlen + clen > cd_size) return bad(err, not_zip + " (truncated central directory)");
        const std::string name(reinterpret_cast<const char *>(h + kCentralLen), nlen);
        // ZIP64 extended information: the 8-byte values of the fields that read 0xffffffff, in order.
        const uint8_t *x = h + kCentralLen + nlen, *xe = x + xlen;
        while (x + 4 <= xe) {
            const uint16_t id = rd16(x), len = rd16(x + 2);
            const uint8_t *d = x + 4, *de = std::min(d + len, xe);
            if (id == 0x0001) {
                if (usize == 0xffffffffu && d + 8 <= de) usize = rd64(d), d += 8;
                if (csize == 0xffffffffu && d + 8 <= de) csize = rd64(d), d += 8;
                if (local == 0xffffffffu && d + 8 <= de) local = rd64(d), d += 8;
            }
            x += 4 + len;
        }
        pos += kCentralLen + nlen + xlen + clen;
        if (name != want_npy && name != key) continue;
        NpzEntry c;
        c.name = name;
        c.bare = name != want_npy;
        c.method = method;
        c.csize = csize;
        c.usize = usize;
        c.crc = crc;
        c.data_pos = local;  // local header offset for now
        if (flags & 1) c.method = -1;  // encrypted
        // A later entry of the same name replaces an earlier one.
        if (c.bare) bare = c, have_bare = true;
        else npy = c, have_npy = true;
    }
    if (!have_npy && !have_bare) return bad(err, "key `" + key + "` not found");
    e = have_npy ? npy : bare;
    if (e.method == -1) return bad(err, "entry `" + e.name + "` is encrypted");
    if (e.method != 0 && e.method != 8)
        return bad(err, "entry `" + e.name + "` uses compression method " + std::to_string(e.method) +
                            " (stored and deflate are read)");
    uint8_t lh[kLocalLen];
    if (e.data_pos + kLocalLen > fsize || !pread_exact(fd, lh, kLocalLen, e.data_pos) || rd32(lh) != kSigLocal)
        return bad(err, not_zip + " (bad local header for `" + e.name + "`)");
    e.data_pos += kLocalLen + rd16(lh + 26) + rd16(lh + 28);
    if (e.method == 0 && e.csize != e.usize) return bad(err, "stored entry `" + e.name + "` has unequal sizes");
    if (e.data_pos > fsize || e.csize > fsize - e.data_pos)
        return bad(err, "entry `" + e.name + "` runs past the end of the file");
    return 0;
}

NpzStream::NpzStream(int fd, const NpzEntry &e) : fd_(fd), e_(e) {
    crc_ = (uint32_t)crc32(0L, Z_NULL, 0);
}

NpzStream::~NpzStream() {
    if (zinit_) inflateEnd(static_cast<z_stream *>(zs_));
    delete static_cast<z_stream *>(zs_);
}

int64_t NpzStream::read(uint8_t *dst, size_t n, std::string &err) {
    if (n == 0) return 0;
    if (e_.method == 0) {
        const uint64_t left = e_.usize - out_;
        const size_t take = (size_t)std::min<uint64_t>(left, n);
        if (take == 0) return 0;
        if (!pread_exact(fd_, dst, take, e_.data_pos + out_)) {
            err = "read failed";
            return -1;
        }
        out_ += take;
        crc_ = npz_crc32(crc_, dst, take);
        return (int64_t)take;
    }
    if (!zinit_) {
        zs_ = new z_stream();
        z_stream *z = static_cast<z_stream *>(zs_);
        if (inflateInit2(z, -MAX_WBITS) != Z_OK) {
            err = "inflateInit2 failed";
            return -1;
        }
        zinit_ = true;
        ibuf_.resize(1 << 20);
    }
    z_stream *z = static_cast<z_stream *>(zs_);
    size_t got = 0;
    while (got < n && !zend_) {
        if (z->avail_in == 0 && in_ < e_.csize) {
            const size_t take = (size_t)std::min<uint64_t>(ibuf_.size(), e_.csize - in_);
            if (!pread_exact(fd_, ibuf_.data(), take, e_.data_pos + in_)) {
                err = "read failed";
                return -1;
            }
            in_ += take;
            z->next_in = ibuf_.data();
            z->avail_in = (uInt)take;
        }
        const size_t want = std::min<size_t>(n - got, 1u << 30);
        z->next_out = dst + got;
        z->avail_out = (uInt)want;
        const int r = inflate(z, Z_NO_FLUSH);
        const size_t made = want - z->avail_out;
        got += made;
        if (r == Z_STREAM_END) {
            zend_ = true;
        } else if (r == Z_BUF_ERROR) {  // no progress possible
            if (z->avail_in == 0 && in_ >= e_.csize) {
                err = "deflate stream ends early";
                return -1;
            }
        } else if (r != Z_OK) {
            err = std::string("inflate failed: ") + (z->msg ? z->msg : "corrupt deflate stream");
            return -1;
        }
    }
    crc_ = npz_crc32(crc_, dst, got);
    out_ += got;
    return (int64_t)got;
}

int64_t npy_data_offset(const uint8_t *p, size_t n, int *major) {
    static const uint8_t magic[6] = {0x93, 'N', 'U', 'M', 'P', 'Y'};
    if (n < 10 || memcmp(p, magic, 6) != 0) return -1;
    *major = p[6];
    if (p[6] == 1) return 10 + (int64_t)rd16(p + 8);
    if (n < 12) return -2;
    return 12 + (int64_t)rd32(p + 8);
}

}  // namespace dmc
