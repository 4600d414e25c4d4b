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
void close(Directory* d);

}  // namespace k3x_reader
