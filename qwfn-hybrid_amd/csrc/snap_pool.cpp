// Device-resident pool of saved sequences.
//
// The reference's server sets a sequence aside when the next request does not
// extend it, keeping at most four under a byte cap, least recently used first
// (saved_seq / save_seq / best_saved, tools/qwfn_server.cpp:767-793). On a new
// prompt it restores the longest saved sequence the prompt extends, or resets
// (restore_or_reset, :1380-1400). A fresh prefill that shares a long prefix with
// a saved sequence stops once at the end of that prefix, so the prefix can be
// saved too (shared_prefix_split, :1401-1424; prefill, :1505-1534). Its
// snapshots are host vectors filled over the host link.
//
// Here the snapshots stay in HBM: a save is a device copy of the parts into a
// pool arena, a restore a device copy back. The arena is two halves of
// cap + slack bytes. Entries are placed first-fit in the current half; when
// the free space is fragmented, the live entries are copied contiguously into
// the other half and the halves swap, so no copy ever overlaps itself.
#include "state_internal.h"

#include <algorithm>
#include <memory>
#include <vector>

using namespace qwfn;

namespace {
constexpr size_t  POOL_ALIGN = 256;
constexpr int32_t MAX_ENTRIES = 64;          // the largest max_entries a pool may have
constexpr int32_t SAVE_MIN_TOKENS = 2048;    // qwfn_server.cpp:1385: worth a prefill later
constexpr int32_t SPLIT_MIN_TOKENS = 2048;   // qwfn_server.cpp:1420
constexpr int32_t SPLIT_MIN_TAIL = 16;       // the prompt goes on past the split
constexpr int32_t SPLIT_MIN_AHEAD = 2;       // the split lies past what the engine holds
constexpr size_t  SLACK_PER_ENTRY = (size_t) 1024 * POOL_ALIGN;   // part alignment, up to 1024 parts

size_t align_up(size_t x) { return (x + POOL_ALIGN - 1) / POOL_ALIGN * POOL_ALIGN; }
}  // namespace

struct qwfn_snap_pool {
    struct entry {
        std::vector<int32_t> tok;
        int32_t              n_past = 0;
        std::vector<size_t>  part_bytes;   // the snapshot's part sizes, checked at load
        size_t               bytes = 0;    // state_snapshot::bytes(): the sum of the parts
        size_t               off = 0;      // blob offset in the current half
        size_t               span = 0;     // arena bytes (parts 256-aligned)
    };
    size_t  cap = 0;
    int32_t max_entries = 4;
    int     device = QWFN_LAYOUT_ONLY;
    char *  arena = nullptr;
    size_t  half_bytes = 0;
    int     half = 0;
    std::vector<entry> saved;             // least recently used first

    ~qwfn_snap_pool() {
        device_scope ds(device);
        if (arena) (void) hipFree(arena);
    }
    char * base(int h) const { return arena ? arena + (size_t) h * half_bytes : nullptr; }
    size_t total() const {
        size_t t = 0;
        for (const auto & e : saved) t += e.bytes;
        return t;
    }
};

namespace {

bool extends(const std::vector<int32_t> & t, const int32_t * tok, int32_t n) {
    return (int32_t) t.size() < n && std::equal(t.begin(), t.end(), tok);
}

// Copies the live entries contiguously into the other half and swaps halves.
// Allocates nothing (at most MAX_ENTRIES entries).
// The bookkeeping moves to the other half only once the copy is launched: a
// launch that fails leaves the pool as it was.
int compact(qwfn_snap_pool & P, hipStream_t stream) {
    const int to = 1 - P.half;
    const char * src[MAX_ENTRIES];
    char * dst[MAX_ENTRIES];
    size_t bytes[MAX_ENTRIES];
    size_t off[MAX_ENTRIES];
    int n = 0;
    size_t cur = 0;
    for (size_t k = 0; k < P.saved.size(); k++) {
        const auto & e = P.saved[k];
        if (P.arena) {
            src[n] = P.base(P.half) + e.off;
            dst[n] = P.base(to) + cur;
            bytes[n] = e.span;
            n++;
        }
        off[k] = cur;
        cur += e.span;
    }
    if (n > 0)
        if (int rc = restore_device(src, bytes, dst, n, 1, 0, stream)) return rc;
    for (size_t k = 0; k < P.saved.size(); k++) P.saved[k].off = off[k];
    P.half = to;
    return QWFN_OK;
}

// First fit of `span` bytes in the current half; compacts when fragmented.
// Allocates nothing.
int place(qwfn_snap_pool & P, size_t span, size_t * off, hipStream_t stream) {
    std::pair<size_t, size_t> used[MAX_ENTRIES];
    int n = 0;
    for (const auto & e : P.saved) used[n++] = {e.off, e.off + e.span};
    std::sort(used, used + n);
    size_t at = 0;
    for (int i = 0; i < n; i++) {
        if (used[i].first - at >= span) break;
        at = std::max(at, used[i].second);
    }
    if (at + span <= P.half_bytes) {
        *off = at;
        return QWFN_OK;
    }
    size_t live = 0;
    for (const auto & e : P.saved) live += e.span;
    if (live + span > P.half_bytes) return set_error(QWFN_ENOMEM, "snap_pool: the pool arena cannot hold the snapshot");
    if (int rc = compact(P, stream)) return rc;
    *off = live;
    return QWFN_OK;
}

int pool_states(const qwfn_snap_pool & P, const qwfn_state * const * sts, int32_t n_sts, const char * what) {
    if (int rc = check_states(sts, n_sts, P.device != QWFN_LAYOUT_ONLY, what)) return rc;
    for (int32_t i = 0; i < n_sts; i++) {
        if (P.device != QWFN_LAYOUT_ONLY && sts[i]->device != P.device)
            return set_error(QWFN_EINVAL, std::string(what) + ": the states and the pool are on different devices");
        if (sts[i]->n_past != sts[0]->n_past) return set_error(QWFN_EINVAL, std::string(what) + ": the states disagree on n_past");
    }
    return QWFN_OK;
}

int reset_states(qwfn_state * const * sts, int32_t n_sts, hipStream_t stream) {
    for (int32_t i = 0; i < n_sts; i++) {
        if (sts[i]->dev)
            if (int rc = zero_recurrent(*sts[i], stream)) return rc;
        sts[i]->n_past = 0;
        sts[i]->rb_depth = 0;
    }
    return QWFN_OK;
}

}  // namespace

extern "C" {

int qwfn_snap_pool_create(size_t cap_bytes, int32_t max_entries, int device, qwfn_snap_pool ** out) {
    return ::qwfn::abi_call("snap_pool_create", [&]() -> int {
        if (!out) return set_error(QWFN_EINVAL, "snap_pool_create: NULL out");
        *out = nullptr;
        if (max_entries < 1 || max_entries > MAX_ENTRIES) return set_error(QWFN_EINVAL, "snap_pool_create: max_entries must be in [1, 64]");
        if (device < QWFN_LAYOUT_ONLY) return set_error(QWFN_EINVAL, "snap_pool_create: bad device");
        std::unique_ptr<qwfn_snap_pool> P(new (std::nothrow) qwfn_snap_pool());
        if (!P) return set_error(QWFN_ENOMEM, "snap_pool_create: out of host memory");
        P->cap = cap_bytes;
        P->max_entries = max_entries;
        P->half_bytes = align_up(cap_bytes) + (size_t) max_entries * SLACK_PER_ENTRY;
        P->device = device;
        if (device != QWFN_LAYOUT_ONLY && cap_bytes) {
            device_scope ds(device);
            if (ds.rc) return ds.rc;
            void * p = nullptr;
            if (hipMalloc(&p, 2 * P->half_bytes) != hipSuccess)
                return set_error(QWFN_ENOMEM, "snap_pool_create: no device memory for the pool arena");
            P->arena = (char *) p;
        }
        *out = P.release();
        return QWFN_OK;
    });
}

void qwfn_snap_pool_destroy(qwfn_snap_pool * P) { delete P; }

int32_t qwfn_snap_pool_count(const qwfn_snap_pool * P) { return P ? (int32_t) P->saved.size() : 0; }

size_t qwfn_snap_pool_bytes(const qwfn_snap_pool * P) { return P ? P->total() : 0; }

int qwfn_snap_pool_entry(const qwfn_snap_pool * P, int32_t k, int32_t * n_tok, int32_t * n_past, size_t * bytes,
                         int32_t * tok, int32_t tok_cap) {
    return ::qwfn::abi_call("snap_pool_entry", [&]() -> int {
        if (!P) return set_error(QWFN_EINVAL, "snap_pool_entry: NULL pool");
        if (k < 0 || k >= (int32_t) P->saved.size()) return set_error(QWFN_ERANGE, "snap_pool_entry: no such entry");
        const auto & e = P->saved[(size_t) k];
        if (n_tok) *n_tok = (int32_t) e.tok.size();
        if (n_past) *n_past = e.n_past;
        if (bytes) *bytes = e.bytes;
        if (tok && tok_cap > 0) std::copy(e.tok.begin(), e.tok.begin() + std::min<size_t>(e.tok.size(), (size_t) tok_cap), tok);
        return QWFN_OK;
    });
}

int qwfn_snap_pool_save(qwfn_snap_pool * P, const qwfn_state * const * sts, int32_t n_sts, const int32_t * tok,
                        int32_t n_tok, void * stream) {
    return ::qwfn::abi_call("snap_pool_save", [&]() -> int {
        if (!P || (!tok && n_tok) || n_tok < 0) return set_error(QWFN_EINVAL, "snap_pool_save: bad arguments");
        if (int rc = pool_states(*P, sts, n_sts, "snap_pool_save")) return rc;
        std::vector<qwfn_part> parts;
        std::vector<bool> host_side;
        for (int32_t i = 0; i < n_sts; i++) parts_of(*sts[i], sts[0]->n_past, parts, &host_side);
        qwfn_snap_pool::entry e;
        e.tok.assign(tok, tok + n_tok);
        e.n_past = sts[0]->n_past;
        for (const auto & p : parts) {
            e.part_bytes.push_back(p.bytes);
            e.bytes += p.bytes;
            e.span += align_up(p.bytes);
        }
        if (e.bytes > P->cap) return 0;                  // larger than the cap: not kept
        // Which entries stay: an equal token sequence is replaced, then the
        // oldest go until within the limits. Nothing changes until the
        // snapshot is known to fit the arena and every host allocation is
        // done, so a host allocation failure leaves the pool as it was. A
        // device error after that point (the launch of the compaction copy or
        // of the snapshot's copy) returns with the evicted entries dropped and
        // the new snapshot not added; the entries kept stay valid (a
        // compaction whose launch fails moves nothing).
        const size_t n_old = P->saved.size();
        bool drop[MAX_ENTRIES] = {};
        for (size_t k = 0; k < n_old; k++)
            if (P->saved[k].tok == e.tok) { drop[k] = true; break; }
        size_t total = e.bytes, kept = 1, live = e.span;
        for (size_t k = 0; k < n_old; k++)
            if (!drop[k]) { total += P->saved[k].bytes; kept++; live += P->saved[k].span; }
        for (size_t k = 0; k < n_old && ((int32_t) kept > P->max_entries || total > P->cap); k++)
            if (!drop[k]) { drop[k] = true; total -= P->saved[k].bytes; kept--; live -= P->saved[k].span; }
        if (live > P->half_bytes)
            return set_error(QWFN_ENOMEM, "snap_pool_save: the pool arena cannot hold the snapshot (too many parts); the pool is unchanged");
        P->saved.reserve(n_old + 1);
        std::vector<const char *> src;
        std::vector<char *> dst;
        std::vector<size_t> b;
        src.reserve(parts.size()); dst.reserve(parts.size()); b.reserve(parts.size());
        device_scope ds(P->device);
        if (ds.rc) return ds.rc;
        hipStream_t s = as_stream(stream);
        // from here on nothing allocates
        for (size_t k = n_old; k-- > 0;)
            if (drop[k]) P->saved.erase(P->saved.begin() + (long) k);
        if (int rc = place(*P, e.span, &e.off, s)) return rc;
        if (P->arena) {
            size_t cur = e.off;
            for (const auto & p : parts) {
                src.push_back((const char *) p.data);
                dst.push_back(P->base(P->half) + cur);
                b.push_back(p.bytes);
                cur += align_up(p.bytes);
            }
            if (int rc = copy_parts(src, dst, b, host_side, s)) return rc;
        }
        P->saved.push_back(std::move(e));
        return 1;
    });
}

int32_t qwfn_snap_pool_best(const qwfn_snap_pool * P, const int32_t * tok, int32_t n_tok, int32_t has_images) {
    return ::qwfn::abi_value<int32_t>("snap_pool_best", -1, [&]() -> int32_t {
        if (!P || has_images || !tok || n_tok <= 0) return -1;
        int32_t best = -1;
        for (size_t k = 0; k < P->saved.size(); k++)
            if (extends(P->saved[k].tok, tok, n_tok) && (best < 0 || P->saved[k].tok.size() > P->saved[(size_t) best].tok.size()))
                best = (int32_t) k;
        return best;
    });
}

int qwfn_snap_pool_load(qwfn_snap_pool * P, int32_t k, qwfn_state * const * sts, int32_t n_sts, void * stream) {
    return ::qwfn::abi_call("snap_pool_load", [&]() -> int {
        if (!P) return set_error(QWFN_EINVAL, "snap_pool_load: NULL pool");
        if (k < 0 || k >= (int32_t) P->saved.size()) return set_error(QWFN_ERANGE, "snap_pool_load: no such entry");
        if (int rc = check_states(sts, n_sts, P->device != QWFN_LAYOUT_ONLY, "snap_pool_load")) return rc;
        device_scope ds(P->device);
        if (ds.rc) return ds.rc;
        hipStream_t s = as_stream(stream);
        // snapshot_load resets before it checks the parts (qwfn_engine.cpp:1034-1040)
        if (int rc = reset_states(sts, n_sts, s)) return rc;
        const auto & e = P->saved[(size_t) k];
        std::vector<qwfn_part> parts;
        std::vector<bool> host_side;
        for (int32_t i = 0; i < n_sts; i++) parts_of(*sts[i], e.n_past, parts, &host_side);
        if (parts.size() != e.part_bytes.size()) return set_error(QWFN_ESIZE, "snap_pool_load: part count mismatch");
        for (size_t p = 0; p < parts.size(); p++)
            if (parts[p].bytes != e.part_bytes[p]) return set_error(QWFN_ESIZE, "snap_pool_load: part size mismatch");
        if (P->arena) {
            std::vector<const char *> src;
            std::vector<char *> dst;
            std::vector<size_t> b;
            size_t cur = e.off;
            for (const auto & p : parts) {
                src.push_back(P->base(P->half) + cur);
                dst.push_back((char *) p.data);
                b.push_back(p.bytes);
                cur += align_up(p.bytes);
            }
            if (int rc = copy_parts(src, dst, b, host_side, s)) return rc;
        }
        for (int32_t i = 0; i < n_sts; i++) sts[i]->n_past = e.n_past;
        // most recently used last (qwfn_server.cpp:1395)
        std::rotate(P->saved.begin() + k, P->saved.begin() + k + 1, P->saved.end());
        return QWFN_OK;
    });
}

int32_t qwfn_snap_pool_split(const qwfn_snap_pool * P, const int32_t * prompt, int32_t n_prompt, int32_t n_consumed,
                             int32_t has_images) {
    return ::qwfn::abi_value<int32_t>("snap_pool_split", 0, [&]() -> int32_t {
        if (!P || has_images || !prompt || n_prompt <= 0 || n_consumed >= SAVE_MIN_TOKENS) return 0;
        size_t L = 0;
        for (const auto & sv : P->saved) {
            size_t l = 0;
            const size_t m = std::min(sv.tok.size(), (size_t) n_prompt);
            while (l < m && sv.tok[l] == prompt[l]) l++;
            L = std::max(L, l);
        }
        bool have = false;   // already saved at exactly this point
        for (const auto & sv : P->saved) have |= sv.tok.size() == L && std::equal(sv.tok.begin(), sv.tok.end(), prompt);
        const bool cut = L >= (size_t) SPLIT_MIN_TOKENS && L + SPLIT_MIN_TAIL < (size_t) n_prompt &&
                         (int64_t) L >= (int64_t) n_consumed + SPLIT_MIN_AHEAD && !have;
        return cut ? (int32_t) L : 0;
    });
}

int qwfn_snap_pool_restore_or_reset(qwfn_snap_pool * P, qwfn_state * const * sts, int32_t n_sts, const int32_t * consumed,
                                    int32_t n_consumed, int32_t consumed_has_images, const int32_t * prompt,
                                    int32_t n_prompt, int32_t prompt_has_images, int32_t * n_restored, void * stream) {
    return ::qwfn::abi_call("snap_pool_restore_or_reset", [&]() -> int {
        if (!P || !n_restored || (!consumed && n_consumed) || n_consumed < 0 || (!prompt && n_prompt) || n_prompt < 0)
            return set_error(QWFN_EINVAL, "snap_pool_restore_or_reset: bad arguments");
        if (int rc = pool_states(*P, sts, n_sts, "snap_pool_restore_or_reset")) return rc;
        if (sts[0]->n_past != n_consumed)
            return set_error(QWFN_EINVAL, "snap_pool_restore_or_reset: the consumed tokens are not the states' positions");
        *n_restored = 0;
        // set the current sequence aside if it is worth a prefill later
        // (a save that does not fit is skipped, as the server skips a failed snapshot_save)
        if (n_consumed >= SAVE_MIN_TOKENS && !consumed_has_images) {
            const int rc = qwfn_snap_pool_save(P, sts, n_sts, consumed, n_consumed, stream);
            if (rc < 0 && rc != QWFN_ENOMEM) return rc;
        }
        const int32_t best = qwfn_snap_pool_best(P, prompt, n_prompt, prompt_has_images);
        if (best >= 0) {
            const int32_t n = (int32_t) P->saved[(size_t) best].tok.size();
            const int rc = qwfn_snap_pool_load(P, best, sts, n_sts, stream);
            if (rc == QWFN_OK) {
                *n_restored = n;
                return QWFN_OK;
            }
            if (rc != QWFN_ESIZE) return rc;
        }
        device_scope ds(P->device);
        if (ds.rc) return ds.rc;
        return reset_states(sts, n_sts, as_stream(stream));
    });
}

}  // extern "C"
