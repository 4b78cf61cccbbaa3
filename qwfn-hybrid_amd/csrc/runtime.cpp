// Error strings, per-device status word and library-owned workspace.
#include "qwfn_common.h"

#include <mutex>
#include <vector>

namespace qwfn {

namespace {
thread_local std::string g_last_error;

struct device_slot {
    uint32_t * status = nullptr;   // device word: DEVERR_* bits
    void *     ws     = nullptr;   // library-owned attention workspace
    size_t     ws_bytes = 0;
};
std::mutex               g_mu;
std::vector<device_slot> g_dev;

int current_slot(device_slot ** out) {
    int dev = 0;
    QWFN_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    if ((size_t) dev >= g_dev.size()) g_dev.resize((size_t) dev + 1);
    *out = &g_dev[(size_t) dev];
    return QWFN_OK;
}
}  // namespace

int set_error(int code, const std::string & msg) {
    g_last_error = msg;
    return code;
}

int hip_check(hipError_t e, const char * what) {
    if (e == hipSuccess) return QWFN_OK;
    const int code = (e == hipErrorOutOfMemory) ? QWFN_ENOMEM : QWFN_EDEVICE;
    return set_error(code, std::string(what) + ": " + hipGetErrorString(e));
}

int status_word(uint32_t ** out) {
    device_slot * s = nullptr;
    if (int rc = current_slot(&s)) return rc;
    if (!s->status) {
        void * p = nullptr;
        QWFN_HIP_TRY(hipMalloc(&p, 256));
        QWFN_HIP_TRY(hipMemset(p, 0, 256));
        s->status = static_cast<uint32_t *>(p);
    }
    *out = s->status;
    return QWFN_OK;
}

int library_workspace(size_t bytes, void ** out) {
    device_slot * s = nullptr;
    if (int rc = current_slot(&s)) return rc;
    if (s->ws_bytes < bytes) {
        if (s->ws) {
            QWFN_HIP_TRY(hipDeviceSynchronize());
            QWFN_HIP_TRY(hipFree(s->ws));
            s->ws = nullptr;
            s->ws_bytes = 0;
        }
        size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
        QWFN_HIP_TRY(hipMalloc(&s->ws, want));
        s->ws_bytes = want;
    }
    *out = s->ws;
    return QWFN_OK;
}

}  // namespace qwfn

extern "C" {

int qwfn_abi_version(void) { return QWFN_KV_ABI_VERSION; }

const char * qwfn_last_error(void) { return qwfn::g_last_error.c_str(); }

int qwfn_init(int device) {
    int n = 0;
    QWFN_HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n)
        return qwfn::set_error(QWFN_EINVAL, "qwfn_init: device " + std::to_string(device) + " of " + std::to_string(n));
    QWFN_HIP_TRY(hipSetDevice(device));
    uint32_t * w = nullptr;
    return qwfn::status_word(&w);
}

int qwfn_device_status(void * stream, uint32_t * flags) {
    if (!flags) return qwfn::set_error(QWFN_EINVAL, "qwfn_device_status: flags is NULL");
    uint32_t * w = nullptr;
    if (int rc = qwfn::status_word(&w)) return rc;
    QWFN_HIP_TRY(hipStreamSynchronize(qwfn::as_stream(stream)));
    QWFN_HIP_TRY(hipMemcpy(flags, w, sizeof(uint32_t), hipMemcpyDeviceToHost));
    QWFN_HIP_TRY(hipMemset(w, 0, sizeof(uint32_t)));
    return QWFN_OK;
}

}  // extern "C"
