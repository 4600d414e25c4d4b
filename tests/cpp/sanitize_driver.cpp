// CPU sanitizer driver for the host code that parses untrusted input:
//   sanitize_driver reader FILE...   the K3X reader's open-time checks
//                                    (k3x_reader.cpp) on each file; prints one
//                                    status code per line
//   sanitize_driver sha256 FILE...   the reader's SHA-256 of each file, fed in
//                                    pieces of 1, 63, 64, 65 and 1000 bytes
//                                    in turn (every buffering path); prints
//                                    one hex digest per line
//   sanitize_driver checks SEED N    HipMoeBackend's argument checks
//                                    (k3x_hip_checks.hpp) over N randomised
//                                    views: extents that disagree with their
//                                    spans, products past SIZE_MAX, zero and
//                                    odd sizes, 0xFF scales, non-finite values
// tests/test_sanitizers.py builds it with -fsanitize=address,undefined and
// fails on any sanitizer report.  Exit status 0 when every step ran.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "k3x_hip_checks.hpp"
#include "k3x_reader.hpp"

using namespace k3x_amd;

namespace {

std::uint64_t state = 0;
std::uint64_t next() {  // SplitMix64 (Steele, Lea & Flood 2014)
    std::uint64_t z = (state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

std::size_t pick_extent() {
    static const std::size_t v[] = {0, 1, 2, 3, 16, 31, 32, 33, 64, 96, 128, 256,
                                    (std::size_t)1 << 32, std::numeric_limits<std::size_t>::max() / 2 + 1,
                                    std::numeric_limits<std::size_t>::max()};
    return v[next() % (sizeof(v) / sizeof(v[0]))];
}

constexpr std::size_t kBytes = 1 << 16, kFloats = 1 << 14;
std::vector<std::byte> bytes_buf(kBytes);
std::vector<float> float_buf(kFloats);

// A span over the buffer whose length is either the extents' product (when
// it fits) or some other length.
std::span<const std::byte> byte_span(std::size_t want) {
    const std::size_t n = (next() % 3 && want <= kBytes) ? want : next() % (kBytes + 1);
    return {bytes_buf.data(), n};
}
std::span<const float> float_span(std::size_t want) {
    const std::size_t n = (next() % 3 && want <= kFloats) ? want : next() % (kFloats + 1);
    return {float_buf.data(), n};
}

std::size_t product_or_max(std::size_t a, std::size_t b) {
    return checks::mul_fits(a, b) ? a * b : std::numeric_limits<std::size_t>::max();
}

Mxfp4WeightView mxfp4_view(std::uint64_t id) {
    const std::size_t rows = pick_extent(), cols = pick_extent();
    std::size_t g = pick_extent() % 40;
    if (next() % 2) g = 32;
    const std::size_t el = product_or_max(rows, cols);
    return {id, byte_span(el / 2), byte_span(g ? el / g : 0), rows, cols, g};
}

DenseWeightView dense_view(std::uint64_t id) {
    const std::size_t rows = pick_extent(), cols = pick_extent();
    return {id, float_span(product_or_max(rows, cols)), rows, cols};
}

int run_checks(std::uint64_t seed, long n) {
    state = seed;
    for (auto& b : bytes_buf) b = std::byte(next() & 0xff);
    for (auto& f : float_buf) f = (float)((int)(next() % 2001) - 1000) / 100.0f;
    float_buf[7] = std::numeric_limits<float>::quiet_NaN();
    float_buf[11] = std::numeric_limits<float>::infinity();
    long accepted = 0;
    for (long i = 0; i < n; ++i) {
        const std::size_t in = pick_extent();
        const Mxfp4MlpView e{mxfp4_view(1 + 3 * i), mxfp4_view(2 + 3 * i), mxfp4_view(3 + 3 * i)};
        accepted += checks::valid_mxfp4(in, e.gate);
        accepted += checks::valid_mxfp4_mlp(in, e);
        const DenseMlpView m{dense_view(10), dense_view(11), dense_view(12)};
        accepted += checks::valid_dense(in, m.gate);
        accepted += checks::valid_dense_size(in, m.down);
        accepted += checks::valid_dense_mlp(in, m);
        const ResidentMoeLayerView rv{dense_view(next() % 4), {next() % 4, float_span(pick_extent())},
                                      dense_view(next() % 4), m};
        const Mxfp4MlpView experts[3] = {e, e, e};
        const std::size_t ne = next() % 4;
        accepted += checks::valid_resident_layer(
            float_span(in), rv, std::span<const Mxfp4MlpView>(experts, ne),
            float_span(next() % 4), (float)(next() % 3) * 1e-6f, 1.0f, std::nullopt);
    }
    std::printf("checks: %ld views, %ld accepted\n", n, accepted);
    return 0;
}

}  // namespace

int sha256_files(int argc, char** argv) {
    static const size_t pieces[] = {1, 63, 64, 65, 1000};
    for (int i = 2; i < argc; ++i) {
        FILE* f = std::fopen(argv[i], "rb");
        if (!f) return 1;
        std::vector<uint8_t> data;
        uint8_t chunk[4096];
        size_t n;
        while ((n = std::fread(chunk, 1, sizeof(chunk), f)) > 0) data.insert(data.end(), chunk, chunk + n);
        std::fclose(f);
        k3x_reader::Sha256 h;
        size_t at = 0, k = 0;
        while (at < data.size()) {
            const size_t take = std::min(pieces[k++ % 5], data.size() - at);
            h.update(data.data() + at, take);
            at += take;
        }
        uint8_t out[32];
        h.finish(out);
        for (uint8_t b : out) std::printf("%02x", b);
        std::printf("\n");
    }
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 2 && !std::strcmp(argv[1], "sha256")) return sha256_files(argc, argv);
    if (argc >= 2 && (!std::strcmp(argv[1], "reader") || !std::strcmp(argv[1], "verify"))) {
        // reader: the open status of each file; verify: also the checksum
        // verification of each file that opens (-1 when it does not).
        const bool verify = argv[1][0] == 'v';
        for (int i = 2; i < argc; ++i) {
            k3x_reader::Directory d;
            const int st = k3x_reader::open_checked(&d, argv[i]);
            const int vst = verify ? (st ? -1 : k3x_reader::verify_checksums(d)) : 0;
            k3x_reader::close(&d);
            if (verify)
                std::printf("%d %d\n", st, vst);
            else
                std::printf("%d\n", st);
        }
        return 0;
    }
    if (argc == 4 && !std::strcmp(argv[1], "checks"))
        return run_checks(std::stoull(argv[2]), std::stol(argv[3]));
    std::fprintf(stderr, "usage: %s reader|verify FILE... | checks SEED N\n", argv[0]);
    return 2;
}
