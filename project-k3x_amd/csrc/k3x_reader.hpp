// k3x_reader.hpp -- the K3X file reader's open-time checks, host code only
// (no HIP): the superblock, the four directories and every tensor record's
// extents, with the status codes of runtime/src/reader.cpp:414-560.  The
// device upload of expert records (storage.hip) builds on it; a sanitizer
// build of this file alone runs over corrupted files on the CPU.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace k3x_reader {

struct TensorRecord {
    uint64_t id;
    uint16_t dtype, quant;
    uint8_t rank;
    int32_t layer, expert;
    uint64_t dims[4];
    uint64_t data_offset, data_length, aux_offset, aux_length;
    uint32_t data_crc, aux_crc;
};

struct Directory {
    int fd = -1;
    uint64_t file_length = 0;
    uint64_t optional_features = 0;
    std::vector<TensorRecord> tensors;
    uint64_t dir_offset[4] = {}, dir_length[4] = {};  // tensor, layer, expert, config
    uint8_t directory_sha256[32] = {};                // superblock bytes 168..199
    uint8_t root_sha256[32] = {};                     // superblock bytes 200..231
};

// SHA-256 (FIPS 180-4).  The round constants and initial hash value are
// derived at first use from their definition: the first 32 bits of the
// fractional parts of the cube roots of the first 64 primes, and of the
// square roots of the first 8, each found exactly with integer arithmetic.
class Sha256 {
public:
    Sha256();
    void update(const uint8_t* p, size_t n);
    void finish(uint8_t out[32]);

private:
    void block(const uint8_t* p);
    uint32_t h_[8];
    uint8_t buf_[64];
    size_t used_ = 0;
    uint64_t bytes_ = 0;
};

// CRC32C (Castagnoli, reflected, preset and final inversion; the value of
// runtime/src/crc32c.cpp:22-28).
uint32_t crc32c(const uint8_t* p, size_t n);
// FNV-1a 64 of a tensor name (runtime/src/reader.cpp:405-412).
uint64_t fnv1a64(const std::string& s);
// Reads n bytes at off; false on a short read.
bool read_at(int fd, uint64_t off, size_t n, uint8_t* dst);
// Opens and checks `path`; 0 or a K3X status code (the values of
// k3x::ErrorCode).  On failure the caller still calls close().
int open_checked(Directory* d, const char* path);
// The checks Reader::open makes with VerifyMode::checksums
// (runtime/src/reader.cpp:672-721), in its order: every tensor's data and
// auxiliary CRC32C, the SHA-256 of the four directories concatenated, the
// SHA-256 of the whole file with the root digest (bytes 200..231) and the
// superblock CRC (4092..4095) read as zeros.  0 or a K3X status code.
int verify_checksums(const Directory& d);
void close(Directory* d);

}  // namespace k3x_reader
