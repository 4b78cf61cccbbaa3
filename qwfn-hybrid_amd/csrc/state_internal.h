// Internals of the sequence state shared by seq_state.hip and snap_pool.cpp.
#pragma once

#include "qwfn_common.h"
#include "qwfn_state.h"

#include <vector>

namespace qwfn {

// Makes a device current for the scope of a call and restores the previous one.
struct device_scope {
    int prev = -1;
    int rc = QWFN_OK;
    explicit device_scope(int dev) {
        if (dev < 0) return;
        hipError_t e = hipGetDevice(&prev);
        if (e == hipSuccess && prev != dev) e = hipSetDevice(dev);
        else if (e == hipSuccess) prev = -1;
        if (e != hipSuccess) { rc = hip_check(e, "hipSetDevice"); prev = -1; }
    }
    ~device_scope() { if (prev >= 0) (void) hipSetDevice(prev); }
};


}  // namespace qwfn

// The state object behind the qwfn_state handle.
struct qwfn_state {
    struct entry {
        int32_t kind;
        uint32_t il;
        bool    host;      // in the pinned host arena
        size_t  off;       // offset in its arena (recurrent tensors: in the device arena)
        size_t  bytes;     // ggml_nbytes
        int32_t type;
        int64_t ne[4];
        size_t  nb[4];
    };
    qwfn_state_config cfg{};
    int device = QWFN_LAYOUT_ONLY;
    std::vector<entry> entries;
    std::vector<int> k, v, idx, rs, conv;   // entry index per layer, -1 if absent
    int ple = -1;
    size_t dev_bytes = 0, host_bytes = 0, rec_off = 0, rec_bytes = 0;
    char * dev = nullptr;     // device arena
    char * host = nullptr;    // pinned host arena (host address)
    char * host_dev = nullptr;  // its device-side address
    char * rb = nullptr;      // rollback slots
    int32_t n_past = 0, rb_depth = 0;

    ~qwfn_state() {
        qwfn::device_scope ds(device);
        if (dev) (void) hipFree(dev);
        if (rb) (void) hipFree(rb);
        if (host) (void) hipHostFree(host);
    }
    bool is_attn(uint32_t il) const {
        return cfg.full_attention_interval > 0 && ((il + 1) % cfg.full_attention_interval) == 0;
    }
    // device-visible address of an entry (its arena offset without memory)
    char * addr(const entry & e, int32_t slot) const {
        const size_t off = slot >= 0 ? (size_t) slot * rec_bytes + (e.off - rec_off) : e.off;
        const char * base = slot >= 0 ? rb : e.host ? host_dev : dev;
        return reinterpret_cast<char *>(reinterpret_cast<uintptr_t>(base) + off);
    }
    // row bytes of a positional cache (ggml_row_size(type, ne0 / n_ctx))
    size_t row_bytes(const entry & e) const {
        const int64_t per = e.ne[0] / (int64_t) cfg.n_ctx;
        return (size_t) (per / qwfn::type_blck(e.type)) * qwfn::type_size(e.type);
    }
};


namespace qwfn {

// Zero the recurrent region (one fill kernel).
int zero_recurrent(qwfn_state & st, hipStream_t stream);
// snapshot_parts of one state at n positions, appended to `out`; host_side
// (if not null) records which parts live in host memory.
void parts_of(const qwfn_state & st, int32_t n, std::vector<qwfn_part> & out, std::vector<bool> * host_side);
// Part copies: device-to-device parts in batched kernels, parts that touch host
// memory with the copy engine.
int copy_parts(const std::vector<const char *> & src, const std::vector<char *> & dst, const std::vector<size_t> & bytes,
               const std::vector<bool> & host_side, hipStream_t stream);
// Non-null states (with memory when need_memory) on one device.
int check_states(const qwfn_state * const * sts, int32_t n_sts, bool need_memory, const char * what);

}  // namespace qwfn
