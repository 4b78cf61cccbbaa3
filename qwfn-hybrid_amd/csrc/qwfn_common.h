// Shared host/device definitions of the gfx950 q8_0 KV-cache library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "qwfn_kv.h"

namespace qwfn {

// q8_0: { fp16 d; int8 qs[32]; } -- ggml's block_q8_0 (QK8_0 = 32).
constexpr int QK      = 32;
constexpr int QBLOCK  = 34;

// Device-side error flag bits (qwfn_device_status).
constexpr uint32_t DEVERR_SET_ROWS_INDEX = 1u << 0;
constexpr uint32_t DEVERR_GET_ROWS_INDEX = 1u << 1;

// ---- host-side error plumbing (runtime.cpp) ----
int  set_error(int code, const std::string & msg);
int  hip_check(hipError_t e, const char * what);
// Per-device status word (uint32 flags); created by qwfn_init or on first use.
int  status_word(uint32_t ** out);
// Library-owned workspace of at least `bytes` on the current device.
int  library_workspace(size_t bytes, void ** out);
// Device-to-device copy of n_parts parts into n_slots slots (kv_copy.hip):
// dst is [slots][n_parts], slots slot0 .. slot0+n_slots-1 are written; each
// source byte is read once. Parts that are not 16-byte aligned go bytewise.
int  restore_device(const char * const * src, const size_t * bytes, char * const * dst, int n_parts, int n_slots,
                    int slot0, hipStream_t stream);

inline hipStream_t as_stream(void * s) { return reinterpret_cast<hipStream_t>(s); }

inline bool is_aligned(const void * p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline const char * type_name(int32_t t) {
    switch (t) {
        case QWFN_TYPE_F32:  return "f32";
        case QWFN_TYPE_F16:  return "f16";
        case QWFN_TYPE_Q8_0: return "q8_0";
        case QWFN_TYPE_I32:  return "i32";
        default:             return "?";
    }
}

inline size_t type_size(int32_t t) {
    switch (t) {
        case QWFN_TYPE_F32:  return 4;
        case QWFN_TYPE_F16:  return 2;
        case QWFN_TYPE_Q8_0: return QBLOCK;
        case QWFN_TYPE_I32:  return 4;
        default:             return 0;
    }
}

// Elements per type unit along dim 0 (32 for q8_0).
inline int64_t type_blck(int32_t t) { return t == QWFN_TYPE_Q8_0 ? QK : 1; }

// Byte extent of a view (last byte + 1), ggml_nbytes semantics.
inline size_t view_bytes(const qwfn_tensor & t) {
    for (int i = 0; i < 4; i++) if (t.ne[i] <= 0) return 0;
    size_t n = (size_t) (t.ne[0] / type_blck(t.type)) * t.nb[0];
    for (int i = 1; i < 4; i++) n += (size_t) (t.ne[i] - 1) * t.nb[i];
    return n;
}

}  // namespace qwfn

#define QWFN_HIP_TRY(expr)                                         \
    do {                                                           \
        hipError_t e_ = (expr);                                    \
        if (e_ != hipSuccess) return ::qwfn::hip_check(e_, #expr); \
    } while (0)
