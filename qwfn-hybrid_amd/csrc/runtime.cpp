// Error strings, per-device status word and library-owned workspace.
#include "qwfn_common.h"

#include <cstring>
#include <mutex>

namespace qwfn {

namespace {
// The last error message of this thread. A fixed buffer, so that recording an
// error never allocates (an allocation failure is one of the errors reported).
constexpr size_t ERR_CAP = 1024;
thread_local char g_last_error[ERR_CAP];

struct device_slot {
    uint32_t * status = nullptr;   // device word: DEVERR_* bits
    void *     ws     = nullptr;   // library-owned attention workspace
    size_t     ws_bytes = 0;
};
// One slot per device index, at a fixed address for the life of the process
// (a pointer to a slot stays valid whatever other threads do).
constexpr int MAX_DEVICES = 64;
std::mutex  g_mu;
device_slot g_dev[MAX_DEVICES];

int current_slot(device_slot ** out) {
    int dev = 0;
    QWFN_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return set_error(QWFN_ENOTSUP, "qwfn: device index beyond the library's table");
    *out = &g_dev[dev];
    return QWFN_OK;
}

void copy_msg(size_t at, const char * s) noexcept {
    if (!s) return;
    const size_t n = strnlen(s, ERR_CAP - 1 - at);
    memcpy(g_last_error + at, s, n);
    g_last_error[at + n] = '\0';
}
}  // namespace

int set_error(int code, const char * msg) noexcept {
    copy_msg(0, msg);
    return code;
}

int set_error(int code, const std::string & msg) noexcept { return set_error(code, msg.c_str()); }

int set_error2(int code, const char * what, const char * msg) noexcept {
    copy_msg(0, what);
    copy_msg(strnlen(g_last_error, ERR_CAP - 1), msg);
    return code;
}

int hip_check(hipError_t e, const char * what) noexcept {
    if (e == hipSuccess) return QWFN_OK;
    const int code = (e == hipErrorOutOfMemory) ? QWFN_ENOMEM : QWFN_EDEVICE;
    set_error2(code, what, ": ");
    copy_msg(strnlen(g_last_error, ERR_CAP - 1), hipGetErrorString(e));
    return code;
}

int status_word(uint32_t ** out) {
    device_slot * s = nullptr;
    if (int rc = current_slot(&s)) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!s->status) {
        void * p = nullptr;
        QWFN_HIP_TRY(hipMalloc(&p, 256));
        QWFN_HIP_TRY(hipMemset(p, 0, 256));
        s->status = static_cast<uint32_t *>(p);
    }
    *out = s->status;
    return QWFN_OK;
}

int library_workspace(size_t bytes, hipStream_t stream, void ** out) {
    // The buffer is allocated (and regrown) by the library, so its address must
    // never be recorded into a graph: a later, larger call frees it.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    QWFN_HIP_TRY(hipStreamIsCapturing(stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return set_error(QWFN_EINVAL, "workspace: ws == NULL is not allowed while the stream is being captured; pass a workspace");
    device_slot * s = nullptr;
    if (int rc = current_slot(&s)) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (s->ws_bytes < bytes) {
        if (s->ws) {
            // work already queued on any stream may still use the old buffer
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

const char * qwfn_last_error(void) { return qwfn::g_last_error; }

int qwfn_init(int device) {
    return qwfn::abi_call("qwfn_init", [&]() -> int {
        int n = 0;
        QWFN_HIP_TRY(hipGetDeviceCount(&n));
        if (device < 0 || device >= n)
            return qwfn::set_error(QWFN_EINVAL, "qwfn_init: device " + std::to_string(device) + " of " + std::to_string(n));
        QWFN_HIP_TRY(hipSetDevice(device));
        uint32_t * w = nullptr;
        return qwfn::status_word(&w);
    });
}

int qwfn_device_status(void * stream, uint32_t * flags) {
    return qwfn::abi_call("qwfn_device_status", [&]() -> int {
        if (!flags) return qwfn::set_error(QWFN_EINVAL, "qwfn_device_status: flags is NULL");
        uint32_t * w = nullptr;
        if (int rc = qwfn::status_word(&w)) return rc;
        QWFN_HIP_TRY(hipStreamSynchronize(qwfn::as_stream(stream)));
        QWFN_HIP_TRY(hipMemcpy(flags, w, sizeof(uint32_t), hipMemcpyDeviceToHost));
        QWFN_HIP_TRY(hipMemset(w, 0, sizeof(uint32_t)));
        return QWFN_OK;
    });
}

}  // extern "C"
