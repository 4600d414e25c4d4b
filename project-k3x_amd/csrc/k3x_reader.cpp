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

void close(Directory* d) {
    if (d->fd >= 0) ::close(d->fd);
    d->fd = -1;
}

}  // namespace k3x_reader
