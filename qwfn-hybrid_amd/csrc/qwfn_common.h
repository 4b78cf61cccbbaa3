// Shared host/device definitions of the gfx950 q8_0 KV-cache library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <new>
#include <string>

#include "qwfn_kv.h"

namespace qwfn {

// q8_0: { fp16 d; int8 qs[32]; } -- ggml's block_q8_0 (QK8_0 = 32).
constexpr int QK      = 32;
constexpr int QBLOCK  = 34;

// Device-side error flag bits (qwfn_device_status).
constexpr uint32_t DEVERR_SET_ROWS_INDEX = 1u << 0;
constexpr uint32_t DEVERR_GET_ROWS_INDEX = 1u << 1;

// x / d through m = ceil(2^32 / d): floor(x * m / 2^32) = floor(x / d) while
// x * d < 2^32 (the host checks the ranges of a call); d = 1 needs no m.
__device__ __forceinline__ uint32_t udiv(uint32_t x, uint32_t d, uint32_t m) {
    return d == 1 ? x : __umulhi(x, m);
}
// A pointer the compiler cannot place (one held in a struct of pointers, or
// a select of two) is accessed with flat instructions, which also count on
// the LDS counter, so that an LDS wait (a lane shuffle) waits for them too.
// gptr states that it points to global memory.
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T * gptr(T * p) {
    return (__attribute__((address_space(1))) T *) p;
}
// the m of udiv, on the host
inline uint32_t recip32(int64_t d) {
    return d > 1 ? (uint32_t) (((uint64_t(1) << 32) + (uint64_t) d - 1) / (uint64_t) d) : 0u;
}

// ---- host-side error plumbing (runtime.cpp) ----
// The message goes into a fixed thread-local buffer: recording an error never
// allocates and never throws.
int  set_error(int code, const char * msg) noexcept;
int  set_error(int code, const std::string & msg) noexcept;
int  set_error2(int code, const char * what, const char * msg) noexcept;
int  hip_check(hipError_t e, const char * what) noexcept;
// Per-device status word (uint32 flags); created by qwfn_init or on first use.
int  status_word(uint32_t ** out);
// Library-owned workspace of at least `bytes` on the current device, shared by
// every call on that device that passes no workspace. Refused while `stream`
// is being captured into a graph (a later, larger call frees the buffer).
int  library_workspace(size_t bytes, hipStream_t stream, void ** out);

// The body of an extern "C" entry point: no C++ exception crosses the ABI. A
// host allocation failure returns QWFN_ENOMEM (as the reference's
// engine::snapshot_save returns false on std::bad_alloc, qwfn_engine.cpp:1022-1025);
// any other exception QWFN_EDEVICE.
template <typename F>
int abi_call(const char * what, F && body) noexcept {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        return set_error2(QWFN_ENOMEM, what, ": out of host memory");
    } catch (...) {
        return set_error2(QWFN_EDEVICE, what, ": unexpected host exception");
    }
}
// The same for entry points that return a value (a size, a count): `fallback`
// on an exception, with the error recorded.
template <typename R, typename F>
R abi_value(const char * what, R fallback, F && body) noexcept {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        set_error2(QWFN_ENOMEM, what, ": out of host memory");
    } catch (...) {
        set_error2(QWFN_EDEVICE, what, ": unexpected host exception");
    }
    return fallback;
}
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
