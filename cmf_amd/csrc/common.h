// Shared host/device definitions of the MI355X decode library (libcmfhip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

// TensorDtype ids (cortiq-core/src/types.rs:10-90).
enum : int { DT_Q8ROW = 3, DT_Q4T = 11, DT_Q4TP = 15 };

// Status codes of the C ABI (mirrors gpu.rs:1-12 "false = declined").
enum : int { CMF_OK = 0, CMF_DECLINED = 1, CMF_ERR = -1 };

namespace cmf {

// Thread-local last error, as cortiq_last_error (cortiq-ffi/include/cortiq.h:6-24).
void set_error(const std::string& msg);
int fail(const std::string& msg);  // set_error + return CMF_ERR

#define CMF_HIP(call)                                                                 \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess)                                                         \
            return ::cmf::fail(std::string(#call " failed: ") + hipGetErrorString(e_)); \
    } while (0)

// ---------------------------------------------------------------------------
// Device layouts (all produced at upload time from the quant.rs byte layouts).
//
// Row block = 16 weight rows (the MFMA N dimension).  For every row block the
// weights of one 64-lane wave-load sit in 1 KiB, lane l = 16*s + r holding
// 16 bytes of row r (r = l % 16) at k-slot s = l / 16:
//   q8  : chunk of 64 columns; lane bytes = W[r][64c + 16s .. +15]  (int8)
//   q4t/q4tp : group of 4 tiles (128 columns); lane bytes = 4-byte nibble
//         word s of tiles 4g..4g+3 of row r (tile bytes 4s..4s+3).
// Scales: q8 f32 per row; q4t f16 [rb][tg][r][4 tiles] (128 B per block);
// q4tp u32 per (rb, tg, r) holding four 5-bit rung codes, plus (2^lo, 2^step)
// f32 per row from which every kernel expands the 32-rung ladder as
// t[c] = t[c-1] * ratio (quant.rs:399-410, the format's definition).
// ---------------------------------------------------------------------------
struct DevWeight {
    int dtype = 0;
    int rows = 0, cols = 0;     // logical shape
    int rows_pad = 0;           // multiple of 16
    int kchunks = 0;            // q8: cols_pad/64 ; q4: cols_pad/128
    int cols_pad = 0;
    uint8_t* w = nullptr;       // repacked weight blocks
    void* scale = nullptr;      // q8: f32[rows_pad]; q4t: f16 blocks; q4tp: u32 codes
    float2* rowp = nullptr;     // q4tp: (t0, ratio) per row
    size_t bytes = 0;           // device bytes held
    int device = 0;
};

constexpr int MAXB = 16;  // largest batch a GEMV launch serves

}  // namespace cmf
