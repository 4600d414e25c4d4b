// k3x_reader.cpp -- the K3X reader's open-time checks (host code only).
// The checks follow runtime/src/reader.cpp:414-560 in order, at the same
// byte offsets and with the same status codes, so that a file the reference
// rejects is rejected here with the same code.
#include "k3x_reader.hpp"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <unordered_set>
#include <utility>

#include "../../include/k3x_hip_moe.h"

namespace k3x_reader {

namespace {

template <typename T>
T le(const uint8_t* p, size_t at) {
    T v;
    std::memcpy(&v, p + at, sizeof(T));
    return v;
}

bool range_ok(uint64_t off, uint64_t len, uint64_t file) {
    return off <= file && len <= file - off;
}

bool zero(const uint8_t* p, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (p[i]) return false;
    return true;
}

}  // namespace

uint32_t crc32c(const uint8_t* p, size_t n) {
    static const auto table = [] {
        std::vector<uint32_t> t(256);
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t r = i;
            for (int b = 0; b < 8; ++b) r = (r >> 1) ^ (0x82f63b78u & (0u - (r & 1u)));
            t[i] = r;
        }
        return t;
    }();
    uint32_t r = 0xffffffffu;
    for (size_t i = 0; i < n; ++i) r = table[(r ^ p[i]) & 255] ^ (r >> 8);
    return ~r;
}

namespace {

// floor(x^(1/root) * 2^32) mod 2^32 for a small prime x: the largest m with
// m^root <= x * 2^(32 root), by bisection in 128-bit integers.
uint32_t frac_bits(uint32_t x, int root) {
    using u128 = unsigned __int128;
    const u128 target = (u128)x << (32 * root);
    uint64_t lo = 0, hi = (uint64_t)1 << 40;  // x^(1/root) < 2^8
    while (hi - lo > 1) {
        const uint64_t m = lo + (hi - lo) / 2;
        u128 v = 1;
        for (int i = 0; i < root; ++i) v *= m;
        (v <= target ? lo : hi) = m;
    }
    return (uint32_t)lo;
}

struct Sha256Constants {
    uint32_t k[64], h0[8];
    Sha256Constants() {
        uint32_t primes[64], n = 0;
        for (uint32_t c = 2; n < 64; ++c) {
            bool prime = true;
            for (uint32_t d = 2; d * d <= c && prime; ++d) prime = c % d != 0;
            if (prime) primes[n++] = c;
        }
        for (int i = 0; i < 64; ++i) k[i] = frac_bits(primes[i], 3);
        for (int i = 0; i < 8; ++i) h0[i] = frac_bits(primes[i], 2);
    }
};

const Sha256Constants& sha256_constants() {
    static const Sha256Constants c;
    return c;
}

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

}  // namespace

Sha256::Sha256() { std::memcpy(h_, sha256_constants().h0, sizeof(h_)); }

void Sha256::block(const uint8_t* p) {
    const uint32_t* k = sha256_constants().k;
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
        w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 |
               p[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
        const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
        const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
    for (int t = 0; t < 64; ++t) {
        const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) +
                            k[t] + w[t];
        const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        h = g;
        g = f;
        f = e;
        e = d + t1;
        d = c;
        c = b;
        b = a;
        a = t1 + t2;
    }
    h_[0] += a;
    h_[1] += b;
    h_[2] += c;
    h_[3] += d;
    h_[4] += e;
    h_[5] += f;
    h_[6] += g;
    h_[7] += h;
}

void Sha256::update(const uint8_t* p, size_t n) {
    bytes_ += n;
    if (used_) {
        const size_t take = std::min(n, 64 - used_);
        std::memcpy(buf_ + used_, p, take);
        used_ += take;
        p += take;
        n -= take;
        if (used_ < 64) return;
        block(buf_);
        used_ = 0;
    }
    for (; n >= 64; p += 64, n -= 64) block(p);
    std::memcpy(buf_, p, n);
    used_ = n;
}

void Sha256::finish(uint8_t out[32]) {
    const uint64_t bits = bytes_ * 8;
    const uint8_t one = 0x80, nil = 0;
    update(&one, 1);
    while (used_ != 56) update(&nil, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(len, 8);
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h_[i] >> (24 - 8 * j));
}

uint64_t fnv1a64(const std::string& s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

bool read_at(int fd, uint64_t off, size_t n, uint8_t* dst) {
    while (n) {
        const ssize_t r = pread(fd, dst, n, (off_t)off);
        if (r <= 0) return false;
        dst += r;
        off += (uint64_t)r;
        n -= (size_t)r;
    }
    return true;
}

namespace {

// Directory header: tag, record size, count (reader.cpp:54-65).
bool directory_count(const std::vector<uint8_t>& d, const char* tag, uint32_t rec, uint64_t* n) {
    if (d.size() < 16 || std::memcmp(d.data(), tag, 4) || le<uint32_t>(d.data(), 4) != rec)
        return false;
    const uint64_t c = le<uint64_t>(d.data(), 8);
    if (c > (d.size() - 16) / rec || d.size() != 16 + c * rec) return false;
    *n = c;
    return true;
}

int open_directory(Directory* s, const char* path) {
    s->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (s->fd < 0) return K3X_ERR_IO;
    struct stat st {};
    if (fstat(s->fd, &st)) return K3X_ERR_IO;
    const uint64_t file = (uint64_t)st.st_size;
    if (file < 4096) return K3X_ERR_TRUNCATED_FILE;
    std::vector<uint8_t> sb(4096);
    if (!read_at(s->fd, 0, 4096, sb.data())) return K3X_ERR_TRUNCATED_FILE;
    const uint8_t* b = sb.data();
    if (std::memcmp(b, "K3XCHKPT", 8)) return K3X_ERR_BAD_MAGIC;
    if (le<uint16_t>(b, 8) != 1 || le<uint16_t>(b, 10) != 0 || le<uint32_t>(b, 12) != 4096 ||
        le<uint32_t>(b, 16) != 4096)
        return K3X_ERR_UNSUPPORTED_VERSION;
    if (crc32c(b, 4092) != le<uint32_t>(b, 4092)) return K3X_ERR_SUPERBLOCK_CRC_MISMATCH;
    if (le<uint64_t>(b, 24)) return K3X_ERR_UNSUPPORTED_REQUIRED_FEATURE;  // none supported
    if (!zero(b + 232, 4092 - 232)) return K3X_ERR_INVALID_DIRECTORY;
    s->optional_features = le<uint64_t>(b, 32);
    uint64_t v[10];
    for (int i = 0; i < 10; ++i) v[i] = le<uint64_t>(b, 88 + 8 * i);
    if (le<uint32_t>(b, 20) != 1 || v[9] != file) return K3X_ERR_TRUNCATED_FILE;
    s->file_length = file;
    std::memcpy(s->directory_sha256, b + 168, 32);
    std::memcpy(s->root_sha256, b + 200, 32);
    for (int i = 0; i < 4; ++i) {
        s->dir_offset[i] = v[2 * i];
        s->dir_length[i] = v[2 * i + 1];
    }
    std::vector<uint8_t> dir[4];
    for (int i = 0; i < 4; ++i) {
        const uint64_t off = v[2 * i], len = v[2 * i + 1];
        if (off % 4096 || !range_ok(off, len, file)) return K3X_ERR_INVALID_EXTENT;
        dir[i].resize(len);
        if (!read_at(s->fd, off, len, dir[i].data())) return K3X_ERR_INVALID_DIRECTORY;
    }
    uint64_t nt = 0, nl = 0, ne = 0;
    const std::vector<uint8_t>& cfg = dir[3];
    if (cfg.size() != 256 || !directory_count(dir[0], "TENS", 128, &nt) ||
        !directory_count(dir[1], "LAYR", 64, &nl) || !directory_count(dir[2], "EXPT", 64, &ne) ||
        le<uint32_t>(cfg.data(), 8) != nl || !zero(cfg.data() + 112, 144) ||
        (le<uint32_t>(cfg.data(), 108) & ~3u))
        return K3X_ERR_INVALID_DIRECTORY;
    std::vector<std::pair<uint64_t, uint64_t>> ranges{{0, 4096}};
    for (int i = 0; i < 4; ++i) ranges.push_back({v[2 * i], v[2 * i] + v[2 * i + 1]});
    std::unordered_set<uint64_t> ids;
    for (uint64_t i = 0; i < nt; ++i) {
        const uint8_t* r = dir[0].data() + 16 + i * 128;
        TensorRecord t{};
        t.id = le<uint64_t>(r, 0);
        t.dtype = le<uint16_t>(r, 12);
        t.quant = le<uint16_t>(r, 14);
        t.rank = r[16];
        t.layer = (int32_t)le<uint32_t>(r, 20);
        t.expert = (int32_t)le<uint32_t>(r, 24);
        for (int d = 0; d < 4; ++d) t.dims[d] = le<uint64_t>(r, 32 + 8 * d);
        t.data_offset = le<uint64_t>(r, 64);
        t.data_length = le<uint64_t>(r, 72);
        t.aux_offset = le<uint64_t>(r, 88);
        t.aux_length = le<uint64_t>(r, 96);
        t.data_crc = le<uint32_t>(r, 104);
        t.aux_crc = le<uint32_t>(r, 108);
        if (t.rank > 4 || (t.dtype < 1 || t.dtype > 3) || t.quant > 1 || le<uint32_t>(r, 8) ||
            r[17] || le<uint16_t>(r, 18) || le<uint32_t>(r, 28) || !zero(r + 112, 16) ||
            !ids.insert(t.id).second)
            return K3X_ERR_INVALID_DIRECTORY;
        for (int d = t.rank; d < 4; ++d)
            if (t.dims[d]) return K3X_ERR_INVALID_DIRECTORY;
        if (t.data_offset % 4096 || !range_ok(t.data_offset, t.data_length, file) ||
            (t.aux_length && (t.aux_offset % 4096 || !range_ok(t.aux_offset, t.aux_length, file))))
            return K3X_ERR_INVALID_EXTENT;
        if (t.data_length) ranges.push_back({t.data_offset, t.data_offset + t.data_length});
        if (t.aux_length) ranges.push_back({t.aux_offset, t.aux_offset + t.aux_length});
        s->tensors.push_back(t);
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); ++i)
        if (ranges[i].first < ranges[i - 1].second) return K3X_ERR_INVALID_EXTENT;
    return K3X_OK;
}

}  // namespace

int open_checked(Directory* d, const char* path) { return open_directory(d, path); }

int verify_checksums(const Directory& d) {
    std::vector<uint8_t> buf;
    auto read = [&](uint64_t off, uint64_t len) {
        buf.resize(len);
        return read_at(d.fd, off, len, buf.data());
    };
    for (const TensorRecord& t : d.tensors) {
        if (!read(t.data_offset, t.data_length) || crc32c(buf.data(), buf.size()) != t.data_crc)
            return K3X_ERR_DATA_CRC_MISMATCH;
        if (t.aux_length &&
            (!read(t.aux_offset, t.aux_length) || crc32c(buf.data(), buf.size()) != t.aux_crc))
            return K3X_ERR_AUXILIARY_CRC_MISMATCH;
    }
    Sha256 dir;
    for (int i = 0; i < 4; ++i) {
        if (!read(d.dir_offset[i], d.dir_length[i])) return K3X_ERR_IO;
        dir.update(buf.data(), buf.size());
    }
    uint8_t digest[32];
    dir.finish(digest);
    if (std::memcmp(digest, d.directory_sha256, 32)) return K3X_ERR_DIRECTORY_SHA256_MISMATCH;
    Sha256 root;
    constexpr uint64_t kChunk = 1u << 20;
    for (uint64_t at = 0; at < d.file_length; at += kChunk) {
        const uint64_t n = std::min(kChunk, d.file_length - at);
        if (!read(at, n)) return K3X_ERR_TRUNCATED_FILE;
        for (auto [lo, hi] : {std::pair<uint64_t, uint64_t>{200, 232}, {4092, 4096}})
            for (uint64_t i = std::max(lo, at); i < std::min(hi, at + n); ++i) buf[i - at] = 0;
        root.update(buf.data(), n);
    }
    root.finish(digest);
    if (std::memcmp(digest, d.root_sha256, 32)) return K3X_ERR_ROOT_SHA256_MISMATCH;
    return K3X_OK;
}

void close(Directory* d) {
    if (d->fd >= 0) ::close(d->fd);
    d->fd = -1;
}

}  // namespace k3x_reader
