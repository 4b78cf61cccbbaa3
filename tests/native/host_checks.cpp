// Host-side checks of the library's C ABI, built with AddressSanitizer and
// UndefinedBehaviorSanitizer (tests/native/Makefile) and run by
// tests/test_host_native.py. Needs no GPU: it drives the layout-only state
// (QWFN_LAYOUT_ONLY), snapshot part lists, the saved-sequence pool in its
// bookkeeping-only mode, and the host-side validation of the device entry
// points (which reject their arguments before any launch).
//
// It also replaces the global operator new with one that can be told to fail
// after a given number of allocations, and checks that every entry point
// turns a host allocation failure into QWFN_ENOMEM instead of letting the
// exception cross the C boundary (the reference's engine::snapshot_save
// returns false on std::bad_alloc, qwfn_engine.cpp:1022-1025), and that a
// pool save that fails on a host allocation leaves the pool exactly as it was
// (device errors after the last allocation are outside what this checks).
#include "qwfn_kv.h"
#include "qwfn_state.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

// ------------------------------------------------ allocation fault injection

static long g_fail_after = -1;   // < 0: never fail; else the number of allocations still allowed

void * operator new(size_t n) {
    if (g_fail_after == 0) throw std::bad_alloc();
    if (g_fail_after > 0) g_fail_after--;
    void * p = std::malloc(n ? n : 1);
    if (!p) throw std::bad_alloc();
    return p;
}
void * operator new[](size_t n) { return operator new(n); }
void * operator new(size_t n, const std::nothrow_t &) noexcept {
    try {
        return operator new(n);
    } catch (...) {
        return nullptr;
    }
}
void * operator new[](size_t n, const std::nothrow_t & t) noexcept { return operator new(n, t); }
void operator delete(void * p) noexcept { std::free(p); }
void operator delete[](void * p) noexcept { std::free(p); }
void operator delete(void * p, size_t) noexcept { std::free(p); }
void operator delete[](void * p, size_t) noexcept { std::free(p); }

static int g_fail = 0;
#define CHECK(cond)                                                                          \
    do {                                                                                     \
        if (!(cond)) {                                                                       \
            std::fprintf(stderr, "CHECK failed at %s:%d: %s (last error: %s)\n", __FILE__,   \
                         __LINE__, #cond, qwfn_last_error());                                \
            g_fail++;                                                                        \
        }                                                                                    \
    } while (0)

// Runs `call` with the k-th host allocation failing, for k = 0, 1, ... until it
// succeeds: every failing run must return QWFN_ENOMEM with the out-of-memory
// message and pass `unchanged` (the caller's consistency check).
template <typename Call, typename Check>
static int with_failing_allocations(const char * what, Call call, Check unchanged) {
    int failures = 0;
    for (long k = 0; k < 10000; k++) {
        g_fail_after = k;
        const int rc = call();
        g_fail_after = -1;
        if (rc != QWFN_ENOMEM) {
            if (rc < 0) std::fprintf(stderr, "%s: k=%ld rc=%d (%s)\n", what, k, rc, qwfn_last_error());
            CHECK(rc >= 0);
            return failures;
        }
        CHECK(std::strstr(qwfn_last_error(), "out of host memory") != nullptr ||
              std::strstr(qwfn_last_error(), "out of memory") != nullptr);
        CHECK(unchanged());
        failures++;
    }
    CHECK(!"an allocation-failure loop did not end");
    return failures;
}

// ------------------------------------------------------------ the checks

static qwfn_state * layout_state(uint32_t n_ctx, uint32_t n_rollback = 0) {
    qwfn_state_config c;
    qwfn_state_config_default(&c, n_ctx);
    c.n_rollback = n_rollback;
    qwfn_state * st = nullptr;
    CHECK(qwfn_state_create(&c, QWFN_LAYOUT_ONLY, &st) == QWFN_OK && st);
    return st;
}

static void check_state_layout() {
    qwfn_state * st = layout_state(73728, 3);
    char buf[512];
    const int n = qwfn_state_summary(st, buf, sizeof buf);
    CHECK(n > 0 && std::strcmp(buf, "state @ 73728 ctx: KV 0.962593 GB (q8_0), indexer 0.226492 GB, deltanet 113.246 MB "
                                     "(constant), conv 4.79232 MB  =>  total 1.30712 GB on the device") == 0);
    char tiny[8];
    CHECK(qwfn_state_summary(st, tiny, sizeof tiny) == n && std::strlen(tiny) == 7);
    CHECK(qwfn_state_bytes(st) == 1307123712u);
    qwfn_tensor t;
    CHECK(qwfn_state_tensor(st, QWFN_STATE_K, 3, -1, &t) == 1 && t.type == QWFN_TYPE_Q8_0 && t.ne[0] == 512 * 73728);
    CHECK(qwfn_state_tensor(st, QWFN_STATE_K, 0, -1, &t) == 0);   // a DeltaNet layer has no cache
    CHECK(qwfn_state_tensor(st, QWFN_STATE_RS, 0, 2, &t) == 1);
    CHECK(qwfn_state_tensor(st, QWFN_STATE_RS, 0, 3, &t) == QWFN_ERANGE);
    CHECK(qwfn_state_tensor(st, 99, 0, -1, &t) == QWFN_EINVAL);
    // bookkeeping: a verified step of 4 positions leaves 3 rollback slots
    CHECK(qwfn_state_step_done(st, 4, 1) == QWFN_OK && qwfn_state_rollback_depth(st) == 3 && qwfn_state_n_past(st) == 4);
    CHECK(qwfn_state_rollback(st, 4, nullptr) == QWFN_ERANGE);
    CHECK(qwfn_state_step_done(st, 73728, 0) == QWFN_ERANGE);
    CHECK(qwfn_state_reset(st, nullptr) == QWFN_OK && qwfn_state_n_past(st) == 0);
    // snapshot parts: 12 x (K, V, idx) + 36 x (rs, conv) + the PLE history
    const qwfn_state * sts[1] = {st};
    int32_t np = 0;
    CHECK(qwfn_snapshot_parts(sts, 1, 8192, nullptr, 0, &np) == QWFN_OK && np == 109);
    std::vector<qwfn_part> parts((size_t) np);
    CHECK(qwfn_snapshot_parts(sts, 1, 8192, parts.data(), np, &np) == QWFN_OK);
    // per layer: 3 DeltaNet layers (rs, conv) then an attention layer (K, V, idx)
    size_t kv = 0;
    for (int l = 0; l < 12; l++) kv += parts[(size_t) (9 * l + 6)].bytes + parts[(size_t) (9 * l + 7)].bytes;
    CHECK(kv == (size_t) 12 * 8192 * 1088);
    CHECK(parts[8].bytes == (size_t) 8192 * 256);   // indexer keys: 128 f16 per position
    CHECK(qwfn_snapshot_parts(sts, 1, -1, parts.data(), np, &np) == QWFN_EINVAL);
    CHECK(qwfn_snapshot_save(sts, 1, nullptr, nullptr, 0, QWFN_MEM_DEVICE, nullptr, nullptr) == QWFN_EINVAL);
    qwfn_state_destroy(st);
    qwfn_state_config bad;
    qwfn_state_config_default(&bad, 0);
    qwfn_state * none = nullptr;
    CHECK(qwfn_state_create(&bad, QWFN_LAYOUT_ONLY, &none) < 0 && none == nullptr);
}

// A small xorshift for the pool walk (deterministic).
static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(uint32_t n) {
    g_rng ^= g_rng << 13; g_rng ^= g_rng >> 7; g_rng ^= g_rng << 17;
    return (uint32_t) (g_rng % n);
}

struct pool_image {
    int32_t count;
    size_t bytes;
    std::vector<std::vector<int32_t>> toks;
    bool operator==(const pool_image & o) const { return count == o.count && bytes == o.bytes && toks == o.toks; }
};

static pool_image image_of(const qwfn_snap_pool * P) {
    pool_image im{qwfn_snap_pool_count(P), qwfn_snap_pool_bytes(P), {}};
    for (int32_t k = 0; k < im.count; k++) {
        int32_t n = 0;
        qwfn_snap_pool_entry(P, k, &n, nullptr, nullptr, nullptr, 0);
        std::vector<int32_t> t((size_t) n);
        qwfn_snap_pool_entry(P, k, nullptr, nullptr, nullptr, t.data(), n);
        im.toks.push_back(t);
    }
    return im;
}

static void check_pool() {
    qwfn_state * st = layout_state(8192);
    qwfn_state * sts[1] = {st};
    const qwfn_state * csts[1] = {st};
    qwfn_snap_pool * P = nullptr;
    CHECK(qwfn_snap_pool_create(size_t(2) << 30, 4, QWFN_LAYOUT_ONLY, &P) == QWFN_OK);
    qwfn_snap_pool * none = nullptr;
    CHECK(qwfn_snap_pool_create(1 << 20, 0, QWFN_LAYOUT_ONLY, &none) == QWFN_EINVAL && !none);
    CHECK(qwfn_snap_pool_create(1 << 20, 65, QWFN_LAYOUT_ONLY, &none) == QWFN_EINVAL && !none);
    std::vector<int32_t> prompt(6000);
    for (size_t i = 0; i < prompt.size(); i++) prompt[i] = (int32_t) (i * 7 + 1);
    for (int step = 0; step < 400; step++) {
        const int32_t n = 2048 + (int32_t) rnd(3000);
        prompt[(size_t) rnd(n)] = (int32_t) rnd(50);   // sequences share prefixes of varying length
        qwfn_state_reset(st, nullptr);
        CHECK(qwfn_state_step_done(st, n, 0) == QWFN_OK);
        const int op = (int) rnd(4);
        if (op == 0) {
            CHECK(qwfn_snap_pool_save(P, csts, 1, prompt.data(), n, nullptr) >= 0);
        } else if (op == 1) {
            const int32_t b = qwfn_snap_pool_best(P, prompt.data(), n, 0);
            if (b >= 0) CHECK(qwfn_snap_pool_load(P, b, sts, 1, nullptr) == QWFN_OK);
        } else if (op == 2) {
            const int32_t cut = qwfn_snap_pool_split(P, prompt.data(), n, (int32_t) rnd(2048), 0);
            CHECK(cut == 0 || (cut >= 2048 && cut < n));
        } else {
            int32_t restored = -1;
            CHECK(qwfn_snap_pool_restore_or_reset(P, sts, 1, prompt.data(), n, 0, prompt.data(), n + 20, 0, &restored,
                                                  nullptr) == QWFN_OK);
            CHECK(restored >= 0 && restored <= n + 20);
        }
        CHECK(qwfn_snap_pool_count(P) <= 4 && qwfn_snap_pool_bytes(P) <= (size_t(2) << 30));
    }
    // a save that fails to allocate leaves the pool as it was
    qwfn_state_reset(st, nullptr);
    qwfn_state_step_done(st, 5000, 0);
    const pool_image before = image_of(P);
    const int fails = with_failing_allocations(
        "snap_pool_save", [&] { return qwfn_snap_pool_save(P, csts, 1, prompt.data(), 5000, nullptr); },
        [&] { return image_of(P) == before; });
    CHECK(fails >= 3);
    qwfn_snap_pool_destroy(P);
    qwfn_state_destroy(st);
}

static void check_oom_paths() {
    // creating a state, its part list and its summary all allocate
    qwfn_state_config c;
    qwfn_state_config_default(&c, 4096);
    qwfn_state * st = nullptr;
    with_failing_allocations("state_create", [&] { return qwfn_state_create(&c, QWFN_LAYOUT_ONLY, &st); },
                             [&] { return st == nullptr; });
    CHECK(st != nullptr);
    const qwfn_state * sts[1] = {st};
    int32_t np = 0;
    with_failing_allocations("snapshot_parts", [&] { return qwfn_snapshot_parts(sts, 1, 100, nullptr, 0, &np); },
                             [] { return true; });
    char buf[256];
    with_failing_allocations("state_summary", [&] { return qwfn_state_summary(st, buf, sizeof buf) < 0 ? -6 : 0; },
                             [] { return true; });
    // a rejected attention call builds its message; with that failing the call still returns a code
    qwfn_tensor q{}, k{};
    q.data = (void *) 0x1000; q.type = QWFN_TYPE_F16;
    for (long kfail = 0; kfail < 4; kfail++) {
        g_fail_after = kfail;
        const int rc = qwfn_flash_attn_ext_q8_0(&q, &k, &k, nullptr, 1.f, 0.f, 0.f, &q, 1, nullptr, 0, nullptr);
        g_fail_after = -1;
        CHECK(rc == QWFN_EINVAL || rc == QWFN_ENOMEM);
    }
    qwfn_state_destroy(st);
}

static void check_validation() {
    // device entry points reject bad descriptors before touching the device
    qwfn_tensor q{}, kv{}, dst{};
    q.data = (void *) 0x7F0000000000; q.type = QWFN_TYPE_F32;
    q.ne[0] = 256; q.ne[1] = 3; q.ne[2] = 16; q.ne[3] = 1;
    q.nb[0] = 4; q.nb[1] = 1024; q.nb[2] = 3 * 1024; q.nb[3] = 48 * 1024;
    kv = q; kv.type = QWFN_TYPE_Q8_0; kv.ne[1] = 100; kv.ne[2] = 2; kv.nb[0] = 34; kv.nb[1] = 544; kv.nb[2] = 272;
    kv.nb[3] = 544 * 100;
    dst = q;
    CHECK(qwfn_flash_attn_ext_q8_0(&q, &kv, &kv, nullptr, 1.f, 1.f, 0.f, &dst, 1, nullptr, 0, nullptr) == QWFN_ENOTSUP);
    CHECK(qwfn_flash_attn_ext_q8_0(&q, &kv, &kv, nullptr, 1.f, 0.f, 0.f, &dst, 7, nullptr, 0, nullptr) == QWFN_EINVAL);
    qwfn_tensor kbad = kv;
    kbad.ne[0] = 128;
    CHECK(qwfn_flash_attn_ext_q8_0(&q, &kbad, &kbad, nullptr, 1.f, 0.f, 0.f, &dst, 1, nullptr, 0, nullptr) == QWFN_ENOTSUP);
    CHECK(qwfn_fattn_workspace_size(&q, &kbad, &kbad, nullptr) == 0);
    int64_t seq[17] = {};
    qwfn_tensor qb = q;
    qb.ne[3] = 17;
    CHECK(qwfn_flash_attn_ext_q8_0_seq(&qb, &kv, &kv, nullptr, 1.f, 0.f, 0.f, &dst, 1, nullptr, 0, seq, nullptr) < 0);
    CHECK(qwfn_set_rows_q8_0(&kv, &q, &q, 1, nullptr) < 0);   // a 4-D source
    CHECK(qwfn_state_restore(nullptr, nullptr, nullptr, 1, 1, QWFN_SRC_DEVICE, nullptr) == QWFN_EINVAL);
    CHECK(qwfn_causal_mask_f16(nullptr, 4, 4, 0, 8, nullptr) == QWFN_EINVAL);
    CHECK(qwfn_qsa_bucket(100, 0, 10) == 0);
}

int main() {
    check_state_layout();
    check_pool();
    check_oom_paths();
    check_validation();
    if (g_fail) {
        std::fprintf(stderr, "%d host checks failed\n", g_fail);
        return 1;
    }
    std::printf("host checks ok\n");
    return 0;
}
