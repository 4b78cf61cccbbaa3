// q8_0 quantise-on-append into the KV cache: ggml_set_rows / ggml_cpy F32 -> Q8_0.
//
// Reference call sites: qwfn_graph.cpp:370-384 (kv_append, ggml_cpy of T rows at
// n_past), :612-628 (qsa_dec_kv_write, ggml_set_rows at write_idx), :914-921
// (mtp_head_kv). The arithmetic is ggml's quantize_row_q8_0 (x86 or _ref
// variant), bit-exact.
//
// Mapping: one wavefront quantises 8 q8_0 blocks (256 values = one KV head of a
// row) in a single pass. Each lane loads 4 consecutive floats (one 16-byte
// load), 8 lanes form a block, amax is reduced across the 8 lanes with DPP,
// and every lane computes d, 1/d and rounds its 4 values. Lane 0 of a block
// stores the fp16 scale, every lane its 4 quants (2-byte-aligned, because a
// block is 34 bytes).
#include "q8_device.h"
#include "qwfn_common.h"

namespace qwfn {
namespace {

constexpr int APPEND_THREADS = 256;   // 4 waves, 32 blocks per workgroup

struct append_args {
    const char *    src;       // F32 rows
    size_t          src_nb1;
    char *          dst;       // Q8_0 rows
    size_t          dst_nb1;
    int64_t         dst_rows;  // rows addressable in dst (set_rows bound)
    const int32_t * idx;       // set_rows indices (device) or nullptr for cpy
    size_t          idx_nb0;
    int64_t         n;         // rows to write
    int32_t         bpr;       // blocks per row (ne0 / 32)
    int32_t         x86;       // rounding variant
    uint32_t *      status;
};

template <bool VEC4>
__device__ __forceinline__ void append_rows(const append_args & a) {
    const int64_t gblk = (int64_t) blockIdx.x * (APPEND_THREADS / 8) + (threadIdx.x >> 3);
    const int     sub  = threadIdx.x & 7;               // 4-value group within the block
    const int64_t total = a.n * a.bpr;
    // Whole 8-lane groups are either all in range or all out: DPP partners exist.
    const bool    live = gblk < total;
    const int64_t row  = live ? gblk / a.bpr : 0;
    const int     blk  = live ? (int) (gblk - row * a.bpr) : 0;

    int64_t drow = row;
    bool ok = live;
    if (live && a.idx) {
        drow = *(const int32_t *) ((const char *) a.idx + (size_t) row * a.idx_nb0);
        if (drow < 0 || drow >= a.dst_rows) {
            ok = false;
            if (sub == 0) atomicOr(a.status, DEVERR_SET_ROWS_INDEX);
        }
    }

    float x[4] = {0.f, 0.f, 0.f, 0.f};
    if (live) {
        const float * sp = (const float *) (a.src + (size_t) row * a.src_nb1) + blk * QK + sub * 4;
        if (VEC4) {
            const float4 v = *(const float4 *) sp;
            x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) x[j] = sp[j];
        }
    }
    uint16_t d16;
    float    dq;
    const uint32_t q4 = dev::q8_quantize_lane4(x, a.x86 != 0, &d16, &dq);
    if (!ok) return;

    char * bp = a.dst + (size_t) drow * a.dst_nb1 + (size_t) blk * QBLOCK;
    uint16_t * qp = (uint16_t *) (bp + 2 + sub * 4);
    qp[0] = (uint16_t) (q4 & 0xffffu);
    qp[1] = (uint16_t) (q4 >> 16);
    if (sub == 0) *(uint16_t *) bp = d16;
}

template <bool VEC4>
__global__ __launch_bounds__(APPEND_THREADS) void k_append_q8_0(append_args a) {
    append_rows<VEC4>(a);
}

// The K and the V rows of one append in one launch: blockIdx.y picks the tensor.
template <bool VEC4>
__global__ __launch_bounds__(APPEND_THREADS) void k_append_q8_0_kv(append_args k, append_args v) {
    append_rows<VEC4>(blockIdx.y ? v : k);
}

int launch_append(const append_args & a, bool vec4, hipStream_t stream) {
    const int64_t blocks = a.n * a.bpr;
    if (blocks == 0) return QWFN_OK;
    const int64_t grid = (blocks + APPEND_THREADS / 8 - 1) / (APPEND_THREADS / 8);
    if (grid > 0x7fffffff) return set_error(QWFN_EINVAL, "append: too many rows");
    if (vec4) hipLaunchKernelGGL(k_append_q8_0<true>, dim3((unsigned) grid), dim3(APPEND_THREADS), 0, stream, a);
    else      hipLaunchKernelGGL(k_append_q8_0<false>, dim3((unsigned) grid), dim3(APPEND_THREADS), 0, stream, a);
    return hip_check(hipGetLastError(), "append launch");
}

// k and v have the same n and bpr (checked by the callers).
int launch_append_kv(const append_args & k, const append_args & v, bool vec4, hipStream_t stream) {
    const int64_t blocks = k.n * k.bpr;
    if (blocks == 0) return QWFN_OK;
    const int64_t grid = (blocks + APPEND_THREADS / 8 - 1) / (APPEND_THREADS / 8);
    if (grid > 0x7fffffff) return set_error(QWFN_EINVAL, "append: too many rows");
    if (vec4) hipLaunchKernelGGL(k_append_q8_0_kv<true>, dim3((unsigned) grid, 2), dim3(APPEND_THREADS), 0, stream, k, v);
    else      hipLaunchKernelGGL(k_append_q8_0_kv<false>, dim3((unsigned) grid, 2), dim3(APPEND_THREADS), 0, stream, k, v);
    return hip_check(hipGetLastError(), "append launch");
}

int check_src_f32(const qwfn_tensor * src, const char * op) {
    if (!src || !src->data) return set_error(QWFN_EINVAL, std::string(op) + ": src is NULL");
    if (src->type != QWFN_TYPE_F32) return set_error(QWFN_EINVAL, std::string(op) + ": src must be f32, got " + type_name(src->type));
    if (src->nb[0] != 4) return set_error(QWFN_EINVAL, std::string(op) + ": src rows must be contiguous (nb[0] == 4)");
    if (src->ne[2] != 1 || src->ne[3] != 1) return set_error(QWFN_ENOTSUP, std::string(op) + ": src must be 2-D");
    if (src->ne[0] <= 0 || src->ne[0] % QK) return set_error(QWFN_EINVAL, std::string(op) + ": ne[0] must be a positive multiple of 32");
    if (!is_aligned(src->data, 4) || src->nb[1] % 4) return set_error(QWFN_EALIGN, std::string(op) + ": src must be 4-byte aligned");
    return QWFN_OK;
}

int check_dst_q8(const qwfn_tensor * dst, int64_t ne0, const char * op) {
    if (!dst || !dst->data) return set_error(QWFN_EINVAL, std::string(op) + ": dst is NULL");
    if (dst->type != QWFN_TYPE_Q8_0) return set_error(QWFN_EINVAL, std::string(op) + ": dst must be q8_0, got " + type_name(dst->type));
    if (dst->nb[0] != QBLOCK) return set_error(QWFN_EINVAL, std::string(op) + ": dst nb[0] must be 34");
    if (dst->ne[0] != ne0) return set_error(QWFN_EINVAL, std::string(op) + ": dst ne[0] != src ne[0]");
    if (dst->ne[2] != 1 || dst->ne[3] != 1) return set_error(QWFN_ENOTSUP, std::string(op) + ": dst must be 2-D");
    if (!is_aligned(dst->data, 2) || dst->nb[1] % 2) return set_error(QWFN_EALIGN, std::string(op) + ": dst must be 2-byte aligned");
    if (dst->nb[1] < (size_t) (ne0 / QK) * QBLOCK) return set_error(QWFN_EINVAL, std::string(op) + ": dst rows overlap (nb[1] < row size)");
    return QWFN_OK;
}


// Checks one ggml_set_rows(dst, src, idx) and fills its arguments (all but the
// status word, taken once every check of a call has passed).
int set_rows_args(const qwfn_tensor * dst, const qwfn_tensor * src, const qwfn_tensor * idx, int variant,
                  append_args * a, bool * vec4) {
    if (int rc = check_src_f32(src, "set_rows")) return rc;
    if (int rc = check_dst_q8(dst, src->ne[0], "set_rows")) return rc;
    if (!idx || !idx->data) return set_error(QWFN_EINVAL, "set_rows: idx is NULL");
    if (idx->type != QWFN_TYPE_I32) return set_error(QWFN_EINVAL, "set_rows: idx must be i32");
    if (idx->ne[0] != src->ne[1] || idx->ne[1] != 1 || idx->ne[2] != 1 || idx->ne[3] != 1)
        return set_error(QWFN_EINVAL, "set_rows: idx must be [n] with n == src ne[1]");
    if (!is_aligned(idx->data, 4) || idx->nb[0] % 4) return set_error(QWFN_EALIGN, "set_rows: idx must be 4-byte aligned");
    if (variant != QWFN_Q8_REF && variant != QWFN_Q8_X86) return set_error(QWFN_EINVAL, "set_rows: unknown rounding variant");
    *a = append_args{};
    a->src = (const char *) src->data; a->src_nb1 = src->nb[1];
    a->dst = (char *) dst->data;       a->dst_nb1 = dst->nb[1];
    a->dst_rows = dst->ne[1];
    a->idx = (const int32_t *) idx->data; a->idx_nb0 = idx->nb[0];
    a->n = src->ne[1]; a->bpr = (int32_t) (src->ne[0] / QK); a->x86 = variant == QWFN_Q8_X86;
    *vec4 = is_aligned(src->data, 16) && src->nb[1] % 16 == 0;
    return QWFN_OK;
}

// Checks one ggml_cpy(src, dst) F32 -> Q8_0 and fills its arguments (all but
// the status word).
int cpy_args(const qwfn_tensor * src, const qwfn_tensor * dst, int variant, append_args * a, bool * vec4) {
    if (int rc = check_src_f32(src, "cpy")) return rc;
    if (int rc = check_dst_q8(dst, src->ne[0], "cpy")) return rc;
    if (dst->ne[1] != src->ne[1]) return set_error(QWFN_EINVAL, "cpy: dst ne[1] != src ne[1]");
    if (variant != QWFN_Q8_REF && variant != QWFN_Q8_X86) return set_error(QWFN_EINVAL, "cpy: unknown rounding variant");
    *a = append_args{};
    a->src = (const char *) src->data; a->src_nb1 = src->nb[1];
    a->dst = (char *) dst->data;       a->dst_nb1 = dst->nb[1];
    a->dst_rows = dst->ne[1];
    a->idx = nullptr; a->idx_nb0 = 0;
    a->n = src->ne[1]; a->bpr = (int32_t) (src->ne[0] / QK); a->x86 = variant == QWFN_Q8_X86;
    *vec4 = is_aligned(src->data, 16) && src->nb[1] % 16 == 0;
    return QWFN_OK;
}

int same_shape(const qwfn_tensor * k, const qwfn_tensor * v, const char * op) {
    if (k->ne[0] != v->ne[0] || k->ne[1] != v->ne[1])
        return set_error(QWFN_EINVAL, std::string(op) + ": the K and V sources must have the same shape");
    return QWFN_OK;
}

}  // namespace
}  // namespace qwfn

using namespace qwfn;

extern "C" int qwfn_set_rows_q8_0(const qwfn_tensor * dst, const qwfn_tensor * src, const qwfn_tensor * idx,
                                  int variant, void * stream) {
    return ::qwfn::abi_call("set_rows_q8_0", [&]() -> int {
        append_args a;
        bool vec4;
        if (int rc = set_rows_args(dst, src, idx, variant, &a, &vec4)) return rc;
        if (int rc = status_word(&a.status)) return rc;
        return launch_append(a, vec4, as_stream(stream));
    });
}

extern "C" int qwfn_cpy_f32_q8_0(const qwfn_tensor * src, const qwfn_tensor * dst, int variant, void * stream) {
    return ::qwfn::abi_call("cpy_f32_q8_0", [&]() -> int {
        append_args a;
        bool vec4;
        if (int rc = cpy_args(src, dst, variant, &a, &vec4)) return rc;
        if (int rc = status_word(&a.status)) return rc;
        return launch_append(a, vec4, as_stream(stream));
    });
}

extern "C" int qwfn_set_rows_q8_0_kv(const qwfn_tensor * dst_k, const qwfn_tensor * src_k, const qwfn_tensor * dst_v,
                                     const qwfn_tensor * src_v, const qwfn_tensor * idx, int variant, void * stream) {
    return ::qwfn::abi_call("set_rows_q8_0_kv", [&]() -> int {
        append_args k, v;
        bool vk, vv;
        if (int rc = set_rows_args(dst_k, src_k, idx, variant, &k, &vk)) return rc;
        if (int rc = set_rows_args(dst_v, src_v, idx, variant, &v, &vv)) return rc;
        if (int rc = same_shape(src_k, src_v, "set_rows_kv")) return rc;
        if (int rc = status_word(&k.status)) return rc;
        v.status = k.status;
        return launch_append_kv(k, v, vk && vv, as_stream(stream));
    });
}

extern "C" int qwfn_cpy_f32_q8_0_kv(const qwfn_tensor * src_k, const qwfn_tensor * dst_k, const qwfn_tensor * src_v,
                                    const qwfn_tensor * dst_v, int variant, void * stream) {
    return ::qwfn::abi_call("cpy_f32_q8_0_kv", [&]() -> int {
        append_args k, v;
        bool vk, vv;
        if (int rc = cpy_args(src_k, dst_k, variant, &k, &vk)) return rc;
        if (int rc = cpy_args(src_v, dst_v, variant, &v, &vv)) return rc;
        if (int rc = same_shape(src_k, src_v, "cpy_kv")) return rc;
        if (int rc = status_word(&k.status)) return rc;
        v.status = k.status;
        return launch_append_kv(k, v, vk && vv, as_stream(stream));
    });
}
