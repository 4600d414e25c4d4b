// k3x_gemm.hpp -- the wide expert GEMM (many rows per expert: prefill and
// verification windows), shared by the general forward path.
#pragma once

#include <cstdint>

#include "k3x_device.hpp"
#include "k3x_internal.hpp"

namespace k3x_hip {

// One grouped GEMM launch.  Rows of expert e are the CSR rows [offsets[e],
// offsets[e] + counts[e]); the launch's work items are the 128-row chunks
// (e << 16 | chunk) of items[0, *n_items).  With items == nullptr there is
// one "expert" of `tokens` rows at offset 0 (the shared expert) and item c
// is its chunk c.
struct WideGemmArgs {
    const uint8_t* codes;        // expert 0 base of the tile array
    const uint32_t* scales;      // MXFP4 only
    size_t codes_per_expert;     // bytes
    size_t scales_per_expert;    // dwords
    uint32_t kt, ks;             // K tiles (K / 128), scale dword groups
    uint32_t nrb;                // 16-row blocks of the output (N / 16)
    const uint16_t* a;           // activation rows, bf16
    uint32_t a_stride;           // elements per activation row
    uint32_t a_bytes;            // bytes readable from a (loads past it read 0)
    uint32_t kta;                // activation K tiles (0: kt); 2 kt for split [hi | lo]
                                 // rows against the weights repeated along K
    uint32_t gather;             // A row = pair_token[off + m] (1) or off + m (0)
    const uint32_t* items;       // routed: (expert << 16 | chunk) work items
    const uint32_t* n_items;
    const uint32_t* counts;
    const uint32_t* offsets;
    const uint32_t* pair_token;
    const uint32_t* pair_slot;
    uint32_t tokens;
    uint32_t top_k;
    uint16_t* act;               // gate/up output [row][act_stride] bf16
    uint32_t act_stride;
    uint32_t act_lo;             // gate/up: element offset of the lo half in a row (0: none)
    // Routed kinds on the scaled FP4 MFMA: `a` holds q8 rows (two E4M3
    // terms per element, the bf16 row's bytes; k3x_device.hpp) and qs their
    // scales [row][kt] {hi, lo} dwords.  Null: bf16 rows, weights
    // dequantised to bf16.
    const uint32_t* qs;
    uint32_t qs_bytes;           // bytes readable from qs
    float* y;                    // down output [row][y_stride] fp32
    uint32_t y_stride;
    uint32_t scatter;            // y row = token * top_k + slot (1) or off + m (0)
    k3x_dev::GluParams glu;
    const uint32_t* status;
    uint32_t item_class;         // routed kinds: the size class of the launch's items
};

enum WideKind {
    kWideRoutedGateUp = 0,  // MXFP4 gate + up, GLU -> bf16 act
    kWideRoutedDown = 1,    // MXFP4 down -> fp32 y (scattered per pair)
    kWideSharedGateUp = 2,  // bf16 gate + up, GLU -> bf16 act
    kWideSharedDown = 3,    // bf16 down -> fp32 y
};

// Rows per workgroup chunk of the wide GEMM.
constexpr uint32_t kWideRows = 128;
// K tiles (128 K each) in flight per workgroup; every K extent must be a
// multiple of 128 * kWideStages.
constexpr uint32_t kWideStages = 4;

// Output 16-row blocks one workgroup covers for `kind` (the launch needs
// nrb to be a multiple of it).
uint32_t wide_rb_per_block(WideKind kind);

// Size classes of the routed work items: chunks of more than 96 rows (every
// chunk but an expert's last is full), of 65-96, 33-64 and 1-32 rows,
// multiplied as 8, 6, 4 and 2 row tiles of 16.
constexpr uint32_t kWideClasses = 4;

// Enqueues one wide GEMM on `stream` (the context stream when null):
// max_items row chunks x the output row blocks, one workgroup each.  Routed
// kinds: the items of size class item_class (0 .. kWideClasses - 1), listed
// in the class segments the grouping writes (n_items[1 + c] items of class c
// after those of the classes before it), max_items an upper bound of their
// count.  Shared kinds: item_class -1, every 128-row chunk of the batch.
int launch_wide_gemm(k3x_hip_ctx* ctx, WideKind kind, const WideGemmArgs& a, uint32_t max_items,
                     hipStream_t stream = nullptr, int item_class = -1);

// bf16 rows [rows][cols] (row stride `stride` elements) -> q8 rows q
// ([rows][cols] 16-bit units: 2 cols bytes a row) and their scale dwords qs
// [rows][cols / 128][2] (k3x_device.hpp), on `stream` (the context stream
// when null).  cols a multiple of 128.
int launch_q8_rows(k3x_hip_ctx* ctx, const uint16_t* src, uint32_t rows, uint32_t cols,
                   uint32_t stride, uint16_t* q, uint32_t* qs, hipStream_t stream = nullptr);

}  // namespace k3x_hip
