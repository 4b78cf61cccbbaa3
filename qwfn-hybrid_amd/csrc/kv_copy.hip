// Byte-movement kernels of the KV path: raw row gather and snapshot restore.
//
// Gather: ggml_get_rows on the cache viewed as I32 words (qwfn_graph.cpp:638-645)
// copies whole 544-byte rows of selected cells, no dequantisation; the
// per-segment form gathers one KV head's 272-byte half rows from per-head
// index lists. Each lane moves 16 bytes when rows and strides allow it, else 4.
//
// Restore: engine::snapshot_load copies each snapshot part into the state with
// ggml_backend_tensor_set (qwfn_engine.cpp:1039-1042). Here a device-resident
// snapshot is broadcast into n_slots sequence slots by one kernel that reads
// each source byte once and writes it n_slots times.
#include "qwfn_common.h"

#include <algorithm>
#include <vector>

namespace qwfn {
namespace {

constexpr int COPY_THREADS = 256;

// ------------------------------------------------------------------ gather

struct gather_args {
    const char *    src;
    const char *    src2;      // blockIdx.z 1: the second tensor of a pair (V of K and V), same geometry
    char *          dst2;
    size_t          src_row_stride;
    int64_t         src_rows;
    size_t          seg_off;
    size_t          seg_stride;
    const int32_t * idx;       // [n_seg][n_idx]
    int64_t         n_idx;
    char *          dst;
    size_t          dst_row_stride;
    size_t          dst_seg_stride;
    uint32_t        units;     // copy units (16 or 4 bytes) per segment
    uint32_t        units_mul; // recip32(units)
    uint32_t        rows;      // index rows per workgroup (rows * units * units < 2^32 when rows > 1)
    uint32_t *      status;
};

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// stores that do not keep the line in the caches (nothing in the launch reads
// a destination back)
__device__ __forceinline__ void store_nt(uint4 * p, uint4 v) {
    __builtin_nontemporal_store(v4u{v.x, v.y, v.z, v.w}, (v4u *) p);
}


// Workgroup (x, y, z) copies index rows [x rows, (x + 1) rows) of segment y
// of tensor z (src / dst, or src2 / dst2 for a pair); a lane's unit u of the
// workgroup is part u % units of row u / units (32-bit reciprocal division,
// no 64-bit arithmetic per unit).
template <typename U>
__global__ __launch_bounds__(COPY_THREADS) void k_gather(gather_args a) {
    const uint32_t seg = blockIdx.y;
    const int64_t i0 = (int64_t) blockIdx.x * a.rows;
    const int64_t left = a.n_idx - i0;
    const uint32_t nrow = left < (int64_t) a.rows ? (uint32_t) left : a.rows;
    const uint32_t total = nrow * a.units;
    const int32_t * idx = a.idx + (size_t) seg * (size_t) a.n_idx + i0;
    const char * src = (blockIdx.z ? a.src2 : a.src) + a.seg_off + (size_t) seg * a.seg_stride;
    char * dst = (blockIdx.z ? a.dst2 : a.dst) + (size_t) seg * a.dst_seg_stride + (size_t) i0 * a.dst_row_stride;
    for (uint32_t u = threadIdx.x; u < total; u += COPY_THREADS) {
        const uint32_t row = a.rows == 1 ? 0u : udiv(u, a.units, a.units_mul);
        const uint32_t part = u - row * a.units;
        const int32_t r = idx[row];
        if (r < 0 || r >= a.src_rows) {
            if (part == 0) atomicOr(a.status, DEVERR_GET_ROWS_INDEX);
            continue;
        }
        const U * s = (const U *) (src + (size_t) r * a.src_row_stride) + part;
        U * d = (U *) (dst + (size_t) row * a.dst_row_stride) + part;
        *d = *s;   // (plain stores: non-temporal ones ran 8% slower here)
    }
}

// n_t: 1, or 2 for a pair (src2 / dst2 set)
int launch_gather(gather_args a, size_t seg_bytes, int32_t n_seg, int n_t, hipStream_t stream) {
    const bool v16 = seg_bytes % 16 == 0 && a.src_row_stride % 16 == 0 && a.seg_off % 16 == 0 &&
                     a.seg_stride % 16 == 0 && a.dst_row_stride % 16 == 0 && a.dst_seg_stride % 16 == 0 &&
                     is_aligned(a.src, 16) && is_aligned(a.dst, 16) &&
                     (n_t == 1 || (is_aligned(a.src2, 16) && is_aligned(a.dst2, 16)));
    const uint64_t units = seg_bytes / (v16 ? 16 : 4);
    if (a.n_idx == 0) return QWFN_OK;
    if (units >= (uint64_t(1) << 31))
        return set_error(QWFN_ENOTSUP, "gather: rows of 8 GiB or more are not supported");
    if (n_seg > 65535) return set_error(QWFN_ENOTSUP, "gather: at most 65535 segments");
    // one unit per lane (whole rows per workgroup when rows are short): a
    // lane's copy is one index load, one data load and one store, so the
    // workgroups' loads are all in flight at once (several units per lane
    // chain them: 4.24 us against 3.64 us in the kernel for the 64K gather of
    // K and V)
    const uint64_t per_wg = COPY_THREADS;
    const uint64_t rows = std::max<uint64_t>(1, std::min<uint64_t>(per_wg / units, (uint64_t) a.n_idx));
    const uint64_t gx = ((uint64_t) a.n_idx + rows - 1) / rows;
    if (gx >= (uint64_t(1) << 31)) return set_error(QWFN_ENOTSUP, "gather: too many index rows");
    a.units = (uint32_t) units;
    a.units_mul = recip32((int64_t) units);
    a.rows = (uint32_t) rows;
    const dim3 grid((unsigned) gx, (unsigned) n_seg, (unsigned) n_t);
    if (v16) hipLaunchKernelGGL(k_gather<uint4>, grid, dim3(COPY_THREADS), 0, stream, a);
    else     hipLaunchKernelGGL(k_gather<uint32_t>, grid, dim3(COPY_THREADS), 0, stream, a);
    return hip_check(hipGetLastError(), "gather launch");
}

// ------------------------------------------------------------------ restore / copy

// Parts are cut into chunks of CHUNK_UNITS 16-byte units (4 KB). A workgroup
// copies one chunk at a time, so the part a chunk belongs to is the same for
// all its lanes and is looked up with scalar loads of the part table (a
// per-lane search of the table costs several dependent memory loads per unit).
// Measured on the model's 118 MB rollback copy: one unit per lane and up to
// 16384 workgroups stream at 7.1 TB/s; four units per lane and 2048 workgroups
// at 5.3 TB/s.
constexpr int CHUNK_PER_LANE = 1;
constexpr int CHUNK_UNITS = COPY_THREADS * CHUNK_PER_LANE;
constexpr int COPY_GRID = 16384;

constexpr int RESTORE_MAX_PARTS = 16;   // per launch, with up to RESTORE_MAX_SLOTS slots
constexpr int RESTORE_MAX_SLOTS = 8;
constexpr int COPY_MAX_PARTS = 96;      // per launch, one destination

template <int MP, int MS>
struct chunk_args {
    const char * src[MP];
    char *       dst[MS][MP];
    int64_t      units[MP];       // 16-byte units of each part
    int64_t      cstart[MP + 1];  // prefix sum of chunks
    int32_t      n_parts;
    int32_t      n_slots;
};
static_assert(sizeof(chunk_args<COPY_MAX_PARTS, 1>) <= 4096, "the part table travels as kernel arguments");
static_assert(sizeof(chunk_args<RESTORE_MAX_PARTS, RESTORE_MAX_SLOTS>) <= 4096, "the part table travels as kernel arguments");

// Each source unit is read once and stored to every slot.
template <int MP, int MS>
__global__ __launch_bounds__(COPY_THREADS) void k_copy_chunks(chunk_args<MP, MS> a) {
    const int64_t n_chunks = a.cstart[a.n_parts];
    int p = 0;
    for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
        while (a.cstart[p + 1] <= c) p++;
        const int64_t first = (c - a.cstart[p]) * CHUNK_UNITS;
        const int64_t base = first + threadIdx.x;
        const int64_t units = a.units[p];
        const uint4 * src = (const uint4 *) a.src[p];
        if (first + CHUNK_UNITS <= units) {
            // a whole chunk: all loads in flight together (guarded loads would
            // each be waited for before the next)
            uint4 v[CHUNK_PER_LANE];
#pragma unroll
            for (int j = 0; j < CHUNK_PER_LANE; j++) v[j] = src[base + j * COPY_THREADS];
            for (int sl = 0; sl < (MS == 1 ? 1 : a.n_slots); sl++) {
                uint4 * dst = (uint4 *) a.dst[sl][p];
#pragma unroll
                for (int j = 0; j < CHUNK_PER_LANE; j++) store_nt(&dst[base + j * COPY_THREADS], v[j]);
            }
        } else {
            for (int64_t u = base; u < units; u += COPY_THREADS) {   // the part's last chunk
                const uint4 v = src[u];
                for (int sl = 0; sl < (MS == 1 ? 1 : a.n_slots); sl++) store_nt(&((uint4 *) a.dst[sl][p])[u], v);
            }
        }
    }
}

// Byte tails and parts that are not 16-byte aligned.
__global__ __launch_bounds__(COPY_THREADS) void k_restore_bytes(const char * src, char * d0, char * d1, char * d2,
                                                               char * d3, char * d4, char * d5, char * d6, char * d7,
                                                               int32_t n_slots, int64_t n) {
    char * d[RESTORE_MAX_SLOTS] = {d0, d1, d2, d3, d4, d5, d6, d7};
    for (int64_t i = (int64_t) blockIdx.x * COPY_THREADS + threadIdx.x; i < n; i += (int64_t) gridDim.x * COPY_THREADS) {
        const char v = src[i];
        for (int s = 0; s < n_slots; s++) d[s][i] = v;
    }
}

// dst is [slots][n_parts]; writes slots slot0 .. slot0 + ns - 1 (ns <= MS).
template <int MP, int MS>
int copy_batched(const char * const * src, const size_t * bytes, char * const * dst, int n_parts, int slot0, int ns,
                 hipStream_t stream) {
    auto dst_of = [&](int s, int p) { return dst[(size_t) (slot0 + s) * n_parts + p]; };
    int p = 0;
    while (p < n_parts) {
        chunk_args<MP, MS> a{};
        a.n_slots = ns;
        int np = 0;
        int64_t chunks = 0;
        for (; p < n_parts && np < MP; p++) {
            const size_t b = bytes[p];
            bool aligned = is_aligned(src[p], 16);
            for (int s = 0; s < ns; s++) aligned = aligned && is_aligned(dst_of(s, p), 16);
            const size_t main = aligned ? (b / 16) * 16 : 0;
            if (main) {
                a.src[np] = src[p];
                for (int s = 0; s < ns; s++) a.dst[s][np] = dst_of(s, p);
                a.units[np] = (int64_t) (main / 16);
                a.cstart[np] = chunks;
                chunks += (a.units[np] + CHUNK_UNITS - 1) / CHUNK_UNITS;
                np++;
            }
            if (main < b) {
                char * d[RESTORE_MAX_SLOTS] = {};
                for (int s = 0; s < ns; s++) d[s] = dst_of(s, p) + main;
                const int64_t n = (int64_t) (b - main);
                const int64_t grid = std::min<int64_t>((n + COPY_THREADS - 1) / COPY_THREADS, 4096);
                hipLaunchKernelGGL(k_restore_bytes, dim3((unsigned) grid), dim3(COPY_THREADS), 0, stream, src[p] + main,
                                   d[0], d[1], d[2], d[3], d[4], d[5], d[6], d[7], ns, n);
                if (int rc = hip_check(hipGetLastError(), "copy tail launch")) return rc;
            }
        }
        if (np == 0) continue;
        a.n_parts = np;
        a.cstart[np] = chunks;
        const int64_t grid = std::min<int64_t>(chunks, COPY_GRID);
        hipLaunchKernelGGL((k_copy_chunks<MP, MS>), dim3((unsigned) grid), dim3(COPY_THREADS), 0, stream, a);
        if (int rc = hip_check(hipGetLastError(), "copy launch")) return rc;
    }
    return QWFN_OK;
}

}  // namespace

int restore_device(const char * const * src, const size_t * bytes, char * const * dst, int n_parts, int n_slots,
                   int slot0, hipStream_t stream) {
    if (n_slots == 1) return copy_batched<COPY_MAX_PARTS, 1>(src, bytes, dst, n_parts, slot0, 1, stream);
    for (int s0 = 0; s0 < n_slots; s0 += RESTORE_MAX_SLOTS) {
        const int ns = std::min(RESTORE_MAX_SLOTS, n_slots - s0);
        if (int rc = copy_batched<RESTORE_MAX_PARTS, RESTORE_MAX_SLOTS>(src, bytes, dst, n_parts, slot0 + s0, ns, stream))
            return rc;
    }
    return QWFN_OK;
}

}  // namespace qwfn

using namespace qwfn;

extern "C" int qwfn_get_rows_i32(const qwfn_tensor * src, const qwfn_tensor * idx, const qwfn_tensor * dst,
                                 void * stream) {
    return ::qwfn::abi_call("get_rows_i32", [&]() -> int {
        if (!src || !idx || !dst || !src->data || !idx->data || !dst->data)
            return set_error(QWFN_EINVAL, "get_rows: NULL tensor");
        if (src->type != QWFN_TYPE_I32 || idx->type != QWFN_TYPE_I32 || dst->type != QWFN_TYPE_I32)
            return set_error(QWFN_EINVAL, "get_rows: src, idx and dst must be i32");
        if (src->nb[0] != 4 || dst->nb[0] != 4 || idx->nb[0] != 4)
            return set_error(QWFN_EINVAL, "get_rows: rows must be contiguous words");
        if (src->ne[2] != 1 || src->ne[3] != 1 || idx->ne[1] != 1 || idx->ne[2] != 1 || idx->ne[3] != 1 ||
            dst->ne[2] != 1 || dst->ne[3] != 1)
            return set_error(QWFN_ENOTSUP, "get_rows: only 2-D src/dst and 1-D idx are supported");
        if (dst->ne[0] != src->ne[0] || dst->ne[1] != idx->ne[0])
            return set_error(QWFN_EINVAL, "get_rows: dst must be [src ne[0], idx ne[0]]");
        if (!is_aligned(src->data, 4) || !is_aligned(dst->data, 4) || !is_aligned(idx->data, 4) ||
            src->nb[1] % 4 || dst->nb[1] % 4)
            return set_error(QWFN_EALIGN, "get_rows: 4-byte alignment required");
        uint32_t * st = nullptr;
        if (int rc = status_word(&st)) return rc;
        gather_args a{};
        a.src = (const char *) src->data; a.src_row_stride = src->nb[1]; a.src_rows = src->ne[1];
        a.seg_off = 0; a.seg_stride = 0;
        a.idx = (const int32_t *) idx->data; a.n_idx = idx->ne[0];
        a.dst = (char *) dst->data; a.dst_row_stride = dst->nb[1]; a.dst_seg_stride = 0;
        a.status = st;
        return launch_gather(a, (size_t) src->ne[0] * 4, 1, 1, as_stream(stream));
    });
}

extern "C" int qwfn_kv_gather_segments(const void * src, size_t src_row_stride, int64_t src_rows,
                                       size_t seg_off, size_t seg_stride, size_t seg_bytes, int32_t n_seg,
                                       const int32_t * idx, int64_t n_idx,
                                       void * dst, size_t dst_row_stride, size_t dst_seg_stride, void * stream) {
    return ::qwfn::abi_call("kv_gather_segments", [&]() -> int {
        if (!src || !idx || !dst) return set_error(QWFN_EINVAL, "gather_segments: NULL pointer");
        if (n_seg < 1 || n_idx < 0 || src_rows < 0 || seg_bytes == 0)
            return set_error(QWFN_EINVAL, "gather_segments: empty or negative sizes");
        if (seg_bytes % 4 || seg_off % 4 || seg_stride % 4 || src_row_stride % 4 || dst_row_stride % 4 ||
            dst_seg_stride % 4 || !is_aligned(src, 4) || !is_aligned(dst, 4) || !is_aligned(idx, 4))
            return set_error(QWFN_EALIGN, "gather_segments: sizes, offsets and strides must be multiples of 4");
        if (seg_off + (size_t) (n_seg - 1) * seg_stride + seg_bytes > src_row_stride)
            return set_error(QWFN_ERANGE, "gather_segments: segments extend past the source row");
        if (dst_row_stride < seg_bytes) return set_error(QWFN_EINVAL, "gather_segments: dst rows overlap");
        uint32_t * st = nullptr;
        if (int rc = status_word(&st)) return rc;
        gather_args a{};
        a.src = (const char *) src; a.src_row_stride = src_row_stride; a.src_rows = src_rows;
        a.seg_off = seg_off; a.seg_stride = seg_stride;
        a.idx = idx; a.n_idx = n_idx;
        a.dst = (char *) dst; a.dst_row_stride = dst_row_stride; a.dst_seg_stride = dst_seg_stride;
        a.status = st;
        return launch_gather(a, seg_bytes, n_seg, 1, as_stream(stream));
    });
}

extern "C" int qwfn_kv_gather_segments_kv(const void * src_k, const void * src_v, size_t src_row_stride, int64_t src_rows,
                                          size_t seg_off, size_t seg_stride, size_t seg_bytes, int32_t n_seg,
                                          const int32_t * idx, int64_t n_idx, void * dst_k, void * dst_v,
                                          size_t dst_row_stride, size_t dst_seg_stride, void * stream) {
    return ::qwfn::abi_call("kv_gather_segments_kv", [&]() -> int {
        if (!src_k || !src_v || !idx || !dst_k || !dst_v) return set_error(QWFN_EINVAL, "gather_segments_kv: NULL pointer");
        if (n_seg < 1 || n_idx < 0 || src_rows < 0 || seg_bytes == 0)
            return set_error(QWFN_EINVAL, "gather_segments_kv: empty or negative sizes");
        if (seg_bytes % 4 || seg_off % 4 || seg_stride % 4 || src_row_stride % 4 || dst_row_stride % 4 ||
            dst_seg_stride % 4 || !is_aligned(src_k, 4) || !is_aligned(src_v, 4) || !is_aligned(dst_k, 4) ||
            !is_aligned(dst_v, 4) || !is_aligned(idx, 4))
            return set_error(QWFN_EALIGN, "gather_segments_kv: sizes, offsets and strides must be multiples of 4");
        if (seg_off + (size_t) (n_seg - 1) * seg_stride + seg_bytes > src_row_stride)
            return set_error(QWFN_ERANGE, "gather_segments_kv: segments extend past the source row");
        if (dst_row_stride < seg_bytes) return set_error(QWFN_EINVAL, "gather_segments_kv: dst rows overlap");
        // the two destinations' extents must not overlap each other
        const size_t ext = n_idx == 0 ? 0 : (size_t) (n_seg - 1) * dst_seg_stride + (size_t) (n_idx - 1) * dst_row_stride + seg_bytes;
        const char * k0 = (const char *) dst_k, * v0 = (const char *) dst_v;
        if (ext && k0 < v0 + ext && v0 < k0 + ext) return set_error(QWFN_EINVAL, "gather_segments_kv: dst_k and dst_v overlap");
        uint32_t * st = nullptr;
        if (int rc = status_word(&st)) return rc;
        gather_args a{};
        a.src = (const char *) src_k; a.src2 = (const char *) src_v;
        a.src_row_stride = src_row_stride; a.src_rows = src_rows;
        a.seg_off = seg_off; a.seg_stride = seg_stride;
        a.idx = idx; a.n_idx = n_idx;
        a.dst = (char *) dst_k; a.dst2 = (char *) dst_v;
        a.dst_row_stride = dst_row_stride; a.dst_seg_stride = dst_seg_stride;
        a.status = st;
        return launch_gather(a, seg_bytes, n_seg, 2, as_stream(stream));
    });
}

extern "C" int qwfn_state_restore(const void * const * src, const size_t * bytes, void * const * dst,
                                  int32_t n_parts, int32_t n_slots, int32_t src_kind, void * stream) {
    return ::qwfn::abi_call("state_restore", [&]() -> int {
        if (!src || !bytes || !dst) return set_error(QWFN_EINVAL, "state_restore: NULL array");
        if (n_parts < 0 || n_slots < 1) return set_error(QWFN_EINVAL, "state_restore: need n_parts >= 0 and n_slots >= 1");
        if (src_kind != QWFN_SRC_DEVICE && src_kind != QWFN_SRC_HOST)
            return set_error(QWFN_EINVAL, "state_restore: unknown source kind");
        for (int p = 0; p < n_parts; p++) {
            if (bytes[p] && !src[p]) return set_error(QWFN_EINVAL, "state_restore: NULL source part " + std::to_string(p));
            for (int s = 0; s < n_slots; s++)
                if (bytes[p] && !dst[(size_t) s * n_parts + p])
                    return set_error(QWFN_EINVAL, "state_restore: NULL destination part " + std::to_string(p));
        }
        hipStream_t st = as_stream(stream);
        const char * const * s8 = reinterpret_cast<const char * const *>(src);
        char * const * d8 = reinterpret_cast<char * const *>(dst);
        if (src_kind == QWFN_SRC_DEVICE) return restore_device(s8, bytes, d8, n_parts, n_slots, 0, st);
        for (int p = 0; p < n_parts; p++)
            if (bytes[p]) QWFN_HIP_TRY(hipMemcpyAsync(d8[p], s8[p], bytes[p], hipMemcpyHostToDevice, st));
        if (n_slots == 1) return QWFN_OK;
        // Broadcast slot 0 (now on the device) into slots 1..n_slots-1.
        std::vector<const char *> s0(d8, d8 + n_parts);
        return restore_device(s0.data(), bytes, d8, n_parts, n_slots - 1, 1, st);
    });
}
