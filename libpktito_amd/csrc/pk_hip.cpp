/* The runtime behind include/pk_hip.h: device set-up, the upload registry,
 * per-call staging for the host-pointer drop-in, and argument checking for
 * every entry. The kernels are in q8_kernels.hip.
 *
 * The reference's seam (backend/kernels.h:242-278) is synchronous, takes host
 * pointers and is called concurrently from a pool's threads on disjoint
 * output tiles (core/passes.c:60-72). So each host-pointer call takes a
 * context of its own from a pool - a stream and its device staging - for the
 * length of the call, and returns with the results in host memory. Contexts
 * are made on demand and kept for the process, so concurrent calls never
 * share one and no call waits for another's.
 */
#include "pk_hip.h"
#include "q8_internal.h"

#include <algorithm>
#include <cfenv>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <thread>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <shared_mutex>
#include <vector>

struct pk_hip_q8 {
    const int8_t *hq;           /* host PK_Q8 bytes, the registry's key */
    const float *hs;
    uint32_t rows, cols, ku;
    int8_t *w;                  /* device units */
    float *s;                   /* device scales */
};

namespace {

thread_local char g_err[256];
thread_local const char *g_kernel = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(PK_HIP_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

/* A launcher's nonzero return: -2 sizes no kernel takes (nothing launched),
 * otherwise the HIP error the launch left. */
/* A launcher's failure: -2 the sizes fit no kernel; else the launch's own
 * error, which the launchers leave set (they peek at it) and this reads
 * and clears. */
int launch_fail(int r, const char *what) {
    if (r == -2)
        return fail(PK_HIP_EINVAL, "%s: the sizes fit no kernel", what);
    const hipError_t e = hipGetLastError();
    return hip_fail(e == hipSuccess ? hipErrorLaunchFailure : e, what);
}

#define PK_TRY(call)                                          \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return hip_fail(e_, #call);     \
    } while (0)

std::once_flag g_once;
int g_init = PK_HIP_ENODEV;
int g_dev = -1;
char g_init_err[256];

void init_once() {
    const char *off = getenv("PKTITO_HIP_DISABLE");
    if (off && *off && strcmp(off, "0")) {
        snprintf(g_init_err, sizeof g_init_err, "PKTITO_HIP_DISABLE is set");
        g_init = PK_HIP_ENODEV;
        return;
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
        snprintf(g_init_err, sizeof g_init_err, "no HIP device");
        g_init = PK_HIP_ENODEV;
        return;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        dev = 0;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
        snprintf(g_init_err, sizeof g_init_err, "hipGetDeviceProperties failed");
        g_init = PK_HIP_ENODEV;
        return;
    }
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        snprintf(g_init_err, sizeof g_init_err, "device %d is %s, not gfx950", dev, p.gcnArchName);
        g_init = PK_HIP_ENODEV;
        return;
    }
    g_dev = dev;
    g_init = PK_HIP_OK;
    /* the static scratch's address and event on this device, taken once
     * now (a failure here, its HIP error read and cleared, fails only the
     * entry that uses them) */
    int se = 0;
    (void)pkq8::static_scratch(dev, &se);
}

/* ---------------------------------------------------------- registry --- */

std::shared_mutex g_reg_mu;
std::map<uintptr_t, pk_hip_q8 *> g_reg;     /* host start -> matrix */

/* the matrix whose host bytes hold p, or NULL; caller holds g_reg_mu */
pk_hip_q8 *holding(const void *p) {
    const uintptr_t a = (uintptr_t)p;
    auto it = g_reg.upper_bound(a);
    if (it == g_reg.begin())
        return nullptr;
    --it;
    pk_hip_q8 *m = it->second;
    return a < it->first + (uintptr_t)m->rows * m->cols ? m : nullptr;
}

/* whether [p, p + len) shares a byte with an uploaded matrix's host bytes;
 * caller holds g_reg_mu */
bool overlaps(const void *p, size_t len) {
    const uintptr_t a = (uintptr_t)p;
    if (holding(p))
        return true;
    auto it = g_reg.lower_bound(a);         /* a matrix starting inside the range */
    return it != g_reg.end() && it->first < a + len;
}

void free_matrix(pk_hip_q8 *m) {
    (void)hipSetDevice(g_dev);
    (void)hipFree(m->w);
    (void)hipFree(m->s);
    delete m;
}

/* ----------------------------------------------------------- contexts --- */

/* Host memory that a DMA copy reads or writes must be pinned, and the
 * caller's buffers are not (a mapped model file, malloc'd activations); a
 * copy from pageable memory, and worse a pitched one, runs far below the
 * link's rate. So each context holds kSlots pinned slots in a ring: rows are
 * gathered into one on the CPU while the others' DMAs run, and outputs come
 * back the same way in reverse. */
constexpr size_t kSlot = (size_t)4 << 20;
constexpr int kSlots = 4;

struct Ctx {
    hipStream_t stream = nullptr;
    char *dev = nullptr;
    size_t cap = 0;
    char *skw = nullptr;                    /* the split few-frame products' workspace, zeroed */
    size_t skw_cap = 0;
    char *host[kSlots] = {};
    hipEvent_t ev[kSlots] = {};
    bool used[kSlots] = {};                 /* ev[i] was recorded */
};

std::mutex g_ctx_mu;
std::vector<Ctx *> g_idle;

struct Lease {
    Ctx *c = nullptr;
    ~Lease() {
        if (c) {
            std::lock_guard<std::mutex> lk(g_ctx_mu);
            g_idle.push_back(c);
        }
    }
};

int lease(Lease &l) {
    {
        std::lock_guard<std::mutex> lk(g_ctx_mu);
        if (!g_idle.empty()) {
            l.c = g_idle.back();
            g_idle.pop_back();
        }
    }
    PK_TRY(hipSetDevice(g_dev));
    if (!l.c) {
        Ctx *c = new Ctx;
        hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        /* the first slot now, the others when a call first needs them (a
         * context that only ever stages small calls holds one) */
        if (e == hipSuccess)
            e = hipHostMalloc((void **)&c->host[0], kSlot, hipHostMallocDefault);
        for (int i = 0; i < kSlots && e == hipSuccess; i++)
            e = hipEventCreateWithFlags(&c->ev[i], hipEventDisableTiming);
        if (e != hipSuccess) {
            for (int i = 0; i < kSlots; i++) {
                if (c->ev[i]) (void)hipEventDestroy(c->ev[i]);
                if (c->host[i]) (void)hipHostFree(c->host[i]);
            }
            if (c->stream) (void)hipStreamDestroy(c->stream);
            delete c;
            return hip_fail(e, "making a staging context");
        }
        l.c = c;
    }
    return PK_HIP_OK;
}

/* Helper threads for the staging copies of large calls: one thread copies a
 * slot between pinned and pageable memory at ~20-25 GB/s, below the link's
 * rate, so a slot of a large call is split over the caller and up to
 * kCopyHelpers more threads. One call uses them at a time; a call that
 * finds them busy (the reference's pool dealing many small calls at once)
 * copies alone. The helpers are started on first use, sleep on a condition
 * variable between calls, and live until the process ends (never joined:
 * the team is never destroyed). */
constexpr int kCopyHelpers = 7;
constexpr size_t kCopySplit = (size_t)1 << 20;    /* copies from this size up are split */

class CopyTeam {
  public:
    /* f(part) for part in [0, parts), part 0 on the calling thread;
     * false (nothing run) when another call holds the team */
    bool try_run(int parts, const std::function<void(int)> &f) {
        std::unique_lock<std::mutex> own(run_mu_, std::try_to_lock);
        if (!own.owns_lock())
            return false;
        if (!started_) {
            /* a helper that cannot be started leaves the team unusable:
             * every call then copies alone */
            try {
                for (; helpers_ < kCopyHelpers; helpers_++)
                    std::thread([this, i = helpers_] { work(i + 1); }).detach();
            } catch (...) {
            }
            started_ = true;
        }
        if (helpers_ < kCopyHelpers)
            return false;
        {
            std::lock_guard<std::mutex> lk(mu_);
            fn_ = &f;
            parts_ = parts;
            pending_ = parts - 1;
            gen_++;
            gen_atomic_.store(gen_, std::memory_order_release);
        }
        cv_.notify_all();
        f(0);
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [this] { return pending_ == 0; });
        fn_ = nullptr;
        return true;
    }

  private:
    void work(int part) {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            /* a call's next slot comes within tens of microseconds: poll
             * for it a while before sleeping */
            if (gen_ == seen) {
                lk.unlock();
                const auto t0 = std::chrono::steady_clock::now();
                while (gen_atomic_.load(std::memory_order_acquire) == seen &&
                       std::chrono::steady_clock::now() - t0 < std::chrono::microseconds(200))
                    std::this_thread::yield();
                lk.lock();
            }
            cv_.wait(lk, [&] { return gen_ != seen; });
            seen = gen_;
            if (part >= parts_)
                continue;
            const std::function<void(int)> *f = fn_;
            lk.unlock();
            (*f)(part);
            lk.lock();
            if (--pending_ == 0)
                done_.notify_one();
        }
    }
    std::mutex run_mu_, mu_;
    std::condition_variable cv_, done_;
    const std::function<void(int)> *fn_ = nullptr;
    int parts_ = 0, pending_ = 0;
    uint64_t gen_ = 0;
    std::atomic<uint64_t> gen_atomic_{ 0 };
    bool started_ = false;
    int helpers_ = 0;
};

CopyTeam &copy_team() {
    static CopyTeam *t = new CopyTeam;     /* never destroyed: its threads outlive main */
    return *t;
}

/* Bytes [b0, b0 + len) of a T x rowbytes block held with a pitch, to or from
 * dense memory: row by row, one memcpy when the pitch is the row. */
void gather_one(char *dense, const char *src, size_t b0, size_t len, size_t rowbytes, size_t pitch) {
    if (pitch == rowbytes) {
        memcpy(dense, src + b0, len);
        return;
    }
    while (len) {
        const size_t r = b0 / rowbytes, o = b0 % rowbytes, k = std::min(len, rowbytes - o);
        memcpy(dense, src + r * pitch + o, k);
        dense += k;
        b0 += k;
        len -= k;
    }
}

void scatter_one(char *dst, const char *dense, size_t b0, size_t len, size_t rowbytes, size_t pitch) {
    if (pitch == rowbytes) {
        memcpy(dst + b0, dense, len);
        return;
    }
    while (len) {
        const size_t r = b0 / rowbytes, o = b0 % rowbytes, k = std::min(len, rowbytes - o);
        memcpy(dst + r * pitch + o, dense, k);
        dense += k;
        b0 += k;
        len -= k;
    }
}

/* the same, a large one split over the copy team (64-byte aligned parts) */
void split_copy(size_t len, const std::function<void(size_t, size_t)> &part) {
    if (len >= kCopySplit) {
        const int parts = kCopyHelpers + 1;
        const size_t step = ((len + parts - 1) / parts + 63) & ~(size_t)63;
        const std::function<void(int)> f = [&](int p) {
            const size_t o = (size_t)p * step;
            if (o < len)
                part(o, std::min(step, len - o));
        };
        if (copy_team().try_run(parts, f))
            return;
    }
    part(0, len);
}

void gather(char *dense, const char *src, size_t b0, size_t len, size_t rowbytes, size_t pitch) {
    split_copy(len, [&](size_t o, size_t n) { gather_one(dense + o, src, b0 + o, n, rowbytes, pitch); });
}

void scatter(char *dst, const char *dense, size_t b0, size_t len, size_t rowbytes, size_t pitch) {
    split_copy(len, [&](size_t o, size_t n) { scatter_one(dst, dense + o, b0 + o, n, rowbytes, pitch); });
}

/* slot i ready for a new copy: allocated, and its last DMA done */
int slot_free(Ctx *c, int i) {
    if (!c->host[i])
        PK_TRY(hipHostMalloc((void **)&c->host[i], kSlot, hipHostMallocDefault));
    if (c->used[i])
        PK_TRY(hipEventSynchronize(c->ev[i]));
    return PK_HIP_OK;
}

/* nrows rows of rowbytes from host src (a row every pitch bytes; pitch is
 * not read for one row) to dense device memory at dst, on c's stream. */
int h2d(Ctx *c, void *dst, const void *src, size_t rowbytes, size_t nrows, size_t pitch) {
    const size_t total = rowbytes * nrows;
    int e;
    for (size_t b0 = 0, k = 0; b0 < total; b0 += kSlot, k++) {
        const int i = (int)(k % kSlots);
        const size_t len = std::min(kSlot, total - b0);
        if ((e = slot_free(c, i)))
            return e;
        gather(c->host[i], (const char *)src, b0, len, rowbytes, pitch);
        PK_TRY(hipMemcpyAsync((char *)dst + b0, c->host[i], len, hipMemcpyHostToDevice, c->stream));
        PK_TRY(hipEventRecord(c->ev[i], c->stream));
        c->used[i] = true;
    }
    return PK_HIP_OK;
}

/* The reverse: dense device src, after the stream's earlier work, to host
 * dst with a pitch; returns with the bytes in place. */
int d2h(Ctx *c, void *dst, size_t pitch, const void *src, size_t rowbytes, size_t nrows) {
    const size_t total = rowbytes * nrows, n = (total + kSlot - 1) / kSlot;
    int e;
    auto issue = [&](size_t k) -> int {
        const int i = (int)(k % kSlots);
        const size_t b0 = k * kSlot, len = std::min(kSlot, total - b0);
        if ((e = slot_free(c, i)))
            return e;
        PK_TRY(hipMemcpyAsync(c->host[i], (const char *)src + b0, len, hipMemcpyDeviceToHost, c->stream));
        PK_TRY(hipEventRecord(c->ev[i], c->stream));
        c->used[i] = true;
        return PK_HIP_OK;
    };
    for (size_t k = 0; k < n && k < (size_t)kSlots; k++)
        if ((e = issue(k)))
            return e;
    for (size_t k = 0; k < n; k++) {
        const int i = (int)(k % kSlots);
        const size_t b0 = k * kSlot, len = std::min(kSlot, total - b0);
        PK_TRY(hipEventSynchronize(c->ev[i]));
        scatter((char *)dst, c->host[i], b0, len, rowbytes, pitch);
        if (k + kSlots < n && (e = issue(k + kSlots)))
            return e;
    }
    return PK_HIP_OK;
}

int reserve(Ctx *c, size_t bytes) {
    if (bytes <= c->cap)
        return PK_HIP_OK;
    if (c->dev) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(c->dev);
        c->dev = nullptr;
        c->cap = 0;
    }
    size_t want = bytes + bytes / 4 + (1 << 20);
    if (hipMalloc(&c->dev, want) != hipSuccess) {
        c->dev = nullptr;
        return fail(PK_HIP_ENOMEM, "hipMalloc of %zu bytes of staging failed", want);
    }
    c->cap = want;
    return PK_HIP_OK;
}

size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

/* c's split workspace of at least bytes (made zero once when it grows;
 * every split call leaves its counters zero). */
int reserve_split(Ctx *c, size_t bytes) {
    if (bytes <= c->skw_cap)
        return PK_HIP_OK;
    if (c->skw) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(c->skw);
        c->skw = nullptr;
        c->skw_cap = 0;
    }
    if (hipMalloc(&c->skw, bytes) != hipSuccess) {
        c->skw = nullptr;
        return fail(PK_HIP_ENOMEM, "hipMalloc of %zu bytes of split workspace failed", bytes);
    }
    PK_TRY(hipMemsetAsync(c->skw, 0, bytes, c->stream));
    c->skw_cap = bytes;
    return PK_HIP_OK;
}

int rmode_of_host() {
    switch (fegetround()) {
    case FE_TONEAREST: return 0;
    case FE_UPWARD: return 1;
    case FE_DOWNWARD: return 2;
    case FE_TOWARDZERO: return 3;
    default: return -1;
    }
}

/* The contract of backend/kernels.h:47-58 and :60-83 for an act. */
int check_act(const pk_hip_act *a, bool for_gemm) {
    if (!a)
        return fail(PK_HIP_EINVAL, "act is NULL");
    if (a->T == 0)
        return PK_HIP_OK;
    if (!a->q || !a->d)
        return fail(PK_HIP_EINVAL, "act q or d is NULL");
    if (a->n == 0 || a->qb == 0 || a->n % a->qb)
        return fail(PK_HIP_EINVAL, "qb %u does not divide n %u", a->qb, a->n);
    if (a->n % 16 || a->qb % 16)
        return fail(PK_HIP_EINVAL, "n %u and qb %u must be multiples of 16", a->n, a->qb);
    if (for_gemm) {
        if (a->n % 32)
            return fail(PK_HIP_EINVAL, "gemm_q8 takes n a multiple of 32, not %u", a->n);
        if (a->qb != a->n && a->qb % 32)
            return fail(PK_HIP_EINVAL, "gemm_q8 takes blocks of a multiple of 32, not %u", a->qb);
        if (a->n > 16384)
            return fail(PK_HIP_EINVAL, "n %u is over 16384", a->n);
    }
    return PK_HIP_OK;
}

int launch_quant(pk_hip_act *a, const float *x, size_t xs, hipStream_t s, int rmode = 0) {
    const char *name = "";
    if (const int r = rmode ? pkq8::launch_quantize_directed(a->q, a->d, x, xs, a->n, a->qb, a->T, rmode, s, &name)
                            : pkq8::launch_quantize(a->q, a->d, x, xs, a->n, a->qb, a->T, s, &name))
        return launch_fail(r, "quantize launch");
    g_kernel = name;
    return PK_HIP_OK;
}

/* The whole of matrix m times the packed activations qp of a, the outputs
 * SiLU'd and quantized in blocks of oqb into the packed copy oqp and od (the
 * up product and siluq of core/encoder.c:130-156 in one launch). Returns 0
 * launched, 1 where the tiling has no such epilogue (nothing launched), or
 * minus an error code. */
int launch_product_siluq(const pk_hip_q8 *m, const pk_hip_act *a, const int8_t *qp, int8_t *oqp, float *od,
                         uint32_t oqb, hipStream_t s) {
    pkq8::GemmArgs g;
    g.w = m->w;
    g.wstride = (uint64_t)(m->rows / 16) * pkq8::kUnitBytes;
    g.ws = m->s;
    g.bias = nullptr;
    g.rows = m->rows;
    g.n = a->n;
    g.ku = m->ku;
    g.kr = pkq8::units_with_data(m->cols);
    g.qb = a->qb;
    g.nb = a->n / a->qb;
    g.add = 0;
    g.rmode = 0;
    g.oqp = oqp;
    g.od = od;
    g.oqb = oqb;
    pkq8::SegTable tab;
    tab.nseg = 1;
    tab.s[0] = pkq8::Seg{ nullptr, qp, a->d, 0, (uint64_t)pkq8::packed_groups(a->T) * pkq8::kUnitBytes, a->T, 0 };
    const char *name = "";
    const int r = pkq8::launch_gemm(g, tab, s, &name);
    if (r == -3)
        return 1;
    if (r)
        return -launch_fail(r, "gemm_q8 silu-quantized launch");
    g_kernel = name;
    return 0;
}

int launch_product(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                   const float *ws, const float *bias, const pk_hip_act *a, int add, int rmode,
                   hipStream_t s, const int8_t *qp = nullptr, void *skw = nullptr) {
    pkq8::GemmArgs g;
    g.w = m->w + (size_t)(r0 / 16) * pkq8::kUnitBytes;
    g.wstride = (uint64_t)(m->rows / 16) * pkq8::kUnitBytes;
    g.ws = ws;
    g.bias = bias;
    g.rows = rows;
    g.n = a->n;
    g.ku = m->ku;
    g.kr = pkq8::units_with_data(m->cols);
    g.qb = a->qb;
    g.nb = a->n / a->qb;
    g.add = add;
    g.rmode = rmode;
    g.skw = skw;
    pkq8::SegTable tab;
    tab.nseg = 1;
    tab.s[0] = pkq8::Seg{ out, qp ? qp : a->q, a->d, (uint64_t)os,
                          qp ? (uint64_t)pkq8::packed_groups(a->T) * pkq8::kUnitBytes : 0, a->T, 0 };
    const char *name = "";
    if (const int r = pkq8::launch_gemm(g, tab, s, &name))
        return launch_fail(r, "gemm_q8 launch");
    g_kernel = name;
    return PK_HIP_OK;
}

int check_panel(const pk_hip_q8 *m, uint32_t r0, uint32_t rows, uint32_t n) {
    if (rows % 16 || r0 % 16)
        return fail(PK_HIP_EINVAL, "rows %u and r0 %u must be multiples of 16", rows, r0);
    if ((uint64_t)r0 + rows > m->rows)
        return fail(PK_HIP_EINVAL, "rows [%u, %u) are outside the matrix's %u", r0, r0 + rows, m->rows);
    if (n != m->cols)
        return fail(PK_HIP_EINVAL, "act n %u is not the matrix's %u inputs", n, m->cols);
    return PK_HIP_OK;
}

}  // namespace

/* ================================================================ ABI === */

extern "C" {

const char *pk_hip_strerror(int err) {
    switch (err) {
    case PK_HIP_OK: return "ok";
    case PK_HIP_EINVAL: return "invalid argument";
    case PK_HIP_ENODEV: return "no usable gfx950 device";
    case PK_HIP_ENOMEM: return "out of device memory";
    case PK_HIP_EDEVICE: return "HIP error";
    case PK_HIP_ENOTUP: return "matrix not uploaded";
    case PK_HIP_EROUND: return "unsupported rounding mode";
    case PK_HIP_ETIMEOUT: return "a bounded wait on the device ran out";
    default: return "unknown error";
    }
}

const char *pk_hip_last_error(void) { return g_err; }

const char *pk_hip_last_kernel(void) { return g_kernel; }

int pk_hip_tilings(void) { return pkq8::ring_count(); }

const char *pk_hip_tiling_name(int index) { return pkq8::ring_name(index); }

int pk_hip_force_tiling(int index) { return pkq8::set_ring(index); }

int pk_hip_force_split(int splits) { return pkq8::set_skinny_split(splits); }

size_t pk_hip_gemm_workspace(uint32_t rows) { return pkq8::skinny_workspace_bytes(rows); }

int pk_hip_force_quantize(int kind) { return pkq8::set_quant_kernel(kind); }

int pk_hip_force_attention(int valu) { return pkq8::set_attention_kernels(valu); }

int pk_hip_force_search_resident(int on) { return pkq8::set_search_resident(on != 0) ? 1 : 0; }

int pk_hip_init(void) {
    std::call_once(g_once, init_once);
    if (g_init != PK_HIP_OK)
        return fail(g_init, "%s", g_init_err);
    return PK_HIP_OK;
}

int pk_hip_upload_q8(const int8_t *q, const float *s, uint32_t rows, uint32_t cols) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!q || !s)
        return fail(PK_HIP_EINVAL, "upload: q or s is NULL");
    if (rows == 0 || rows % 16 || cols == 0 || cols % 32 || cols > 16384)
        return fail(PK_HIP_EINVAL, "upload: a q8 matrix is 16 rows by 32 inputs at a time, at most "
                                   "16384 inputs; not %u x %u", rows, cols);
    {
        std::shared_lock<std::shared_mutex> lk(g_reg_mu);
        if (overlaps(q, (size_t)rows * cols))
            return fail(PK_HIP_EINVAL, "upload: host bytes at %p overlap an uploaded matrix", (const void *)q);
    }
    PK_TRY(hipSetDevice(g_dev));
    pk_hip_q8 *m = new pk_hip_q8{ q, s, rows, cols, pkq8::units_per_panel(cols), nullptr, nullptr };
    const size_t raw = (size_t)rows * cols;
    const size_t packed = (size_t)(rows / 16) * m->ku * pkq8::kUnitBytes;
    int8_t *tmp = nullptr;
    hipError_t he = hipMalloc(&tmp, raw);
    if (he == hipSuccess) he = hipMalloc(&m->w, packed);
    if (he == hipSuccess) he = hipMalloc(&m->s, rows * sizeof(float));
    if (he != hipSuccess) {
        (void)hipFree(tmp);
        (void)hipFree(m->w);
        (void)hipFree(m->s);
        delete m;
        return fail(PK_HIP_ENOMEM, "upload: hipMalloc failed for a %u x %u matrix", rows, cols);
    }
    he = hipMemcpy(tmp, q, raw, hipMemcpyHostToDevice);
    if (he == hipSuccess) he = hipMemcpy(m->s, s, rows * sizeof(float), hipMemcpyHostToDevice);
    if (he == hipSuccess && pkq8::launch_repack(m->w, tmp, rows, cols, nullptr)) he = hipGetLastError();
    if (he == hipSuccess) he = hipDeviceSynchronize();
    (void)hipFree(tmp);
    if (he != hipSuccess) {
        free_matrix(m);
        return hip_fail(he, "upload");
    }
    std::unique_lock<std::shared_mutex> lk(g_reg_mu);
    if (overlaps(q, (size_t)rows * cols)) {     /* another thread uploaded these bytes meanwhile */
        lk.unlock();
        free_matrix(m);
        return fail(PK_HIP_EINVAL, "upload: host bytes at %p overlap an uploaded matrix", (const void *)q);
    }
    g_reg[(uintptr_t)q] = m;
    return PK_HIP_OK;
}

int pk_hip_release_q8(const int8_t *q) {
    pk_hip_q8 *m = nullptr;
    {
        std::unique_lock<std::shared_mutex> lk(g_reg_mu);
        auto it = g_reg.find((uintptr_t)q);
        if (it == g_reg.end())
            return fail(PK_HIP_EINVAL, "release: no matrix starts at %p", (const void *)q);
        m = it->second;
        g_reg.erase(it);
    }
    free_matrix(m);
    return PK_HIP_OK;
}

void pk_hip_release_all(void) {
    std::unique_lock<std::shared_mutex> lk(g_reg_mu);
    for (auto &kv : g_reg)
        free_matrix(kv.second);
    g_reg.clear();
}

const pk_hip_q8 *pk_hip_q8_find(const int8_t *q) {
    std::shared_lock<std::shared_mutex> lk(g_reg_mu);
    return holding(q);
}

const float *pk_hip_q8_scales(const pk_hip_q8 *m) { return m ? m->s : nullptr; }
uint32_t pk_hip_q8_rows(const pk_hip_q8 *m) { return m ? m->rows : 0; }
uint32_t pk_hip_q8_cols(const pk_hip_q8 *m) { return m ? m->cols : 0; }

int pk_hip_quantize(pk_hip_act *a, const float *x, size_t xs) {
    int e = pk_hip_init();
    if (e)
        return e;
    if ((e = check_act(a, false)))
        return e;
    if (a->T == 0)
        return PK_HIP_OK;
    if (!x || xs < a->n)
        return fail(PK_HIP_EINVAL, "quantize: x is NULL or its stride %zu is under n %u", xs, a->n);
    /* the calling thread's rounding mode, which the reference's ref follows
     * in both divisions, the product and rintf */
    const int rmode = rmode_of_host();
    if (rmode < 0)
        return fail(PK_HIP_EROUND, "quantize: unknown rounding mode");
    Lease l;
    if ((e = lease(l)))
        return e;
    const size_t n = a->n, T = a->T, nb = n / a->qb;
    const size_t xb = up256(T * n * sizeof(float)), qbytes = up256(T * n);
    if ((e = reserve(l.c, xb + qbytes + up256(T * nb * sizeof(float)))))
        return e;
    float *dx = (float *)l.c->dev;
    int8_t *dq = (int8_t *)(l.c->dev + xb);
    float *dd = (float *)(l.c->dev + xb + qbytes);
    hipStream_t s = l.c->stream;
    if ((e = h2d(l.c, dx, x, n * sizeof(float), T, xs * sizeof(float))))
        return e;
    pk_hip_act da = { dq, dd, a->n, a->qb, a->T };
    if ((e = launch_quant(&da, dx, n, s, rmode)))
        return e;
    if ((e = d2h(l.c, a->q, n, dq, n, T)) || (e = d2h(l.c, a->d, nb * sizeof(float), dd, nb * sizeof(float), T)))
        return e;
    return PK_HIP_OK;
}

int pk_hip_gemm_q8(float *out, size_t os, const int8_t *w, const float *ws, const float *bias,
                   uint32_t rows, const pk_hip_act *a, int add) {
    int e = pk_hip_init();
    if (e)
        return e;
    if ((e = check_act(a, true)))
        return e;
    if (a->T == 0)
        return PK_HIP_OK;          /* no columns: nothing read, nothing written */
    if (!out || !w || !ws)
        return fail(PK_HIP_EINVAL, "gemm_q8: out, w or ws is NULL");
    if (rows % 16)
        return fail(PK_HIP_EINVAL, "gemm_q8: rows %u is not a multiple of 16", rows);
    if (a->T > 1 && os < rows)
        return fail(PK_HIP_EINVAL, "gemm_q8: output stride %zu is under rows %u", os, rows);
    const int rmode = rmode_of_host();
    if (rmode < 0)
        return fail(PK_HIP_EROUND, "gemm_q8: unknown rounding mode");
    /* The registry stays locked (shared) until the call has returned its
     * outputs, so that a release of the matrix waits for it. */
    std::shared_lock<std::shared_mutex> lk(g_reg_mu);
    const pk_hip_q8 *m = holding(w);
    uint32_t r0 = 0;
    if (m) {
        const size_t off = (size_t)(w - m->hq), panel = (size_t)16 * m->cols;
        if (off % panel)
            return fail(PK_HIP_EINVAL, "gemm_q8: w is not at a panel of its matrix");
        r0 = (uint32_t)(off / panel) * 16;
        if ((e = check_panel(m, r0, rows, a->n)))
            return e;
    } else if (a->n > 16384) {
        return fail(PK_HIP_EINVAL, "gemm_q8: n %u over 16384", a->n);
    }
    Lease l;
    if ((e = lease(l)))
        return e;
    const size_t n = a->n, T = a->T, nb = n / a->qb, R = rows;
    const size_t bq = up256(T * n), bd = up256(T * nb * 4), bw = up256(R * 4), bo = up256(T * R * 4);
    /* Weights inside no uploaded matrix (a caller's own buffer, as the
     * reference's checkers pass) are staged for this call alone: their
     * PK_Q8 bytes copied and repacked into the lease's device memory, then
     * the same kernels run. Slower (a copy and a repack a call), same bits. */
    const uint32_t ku = pkq8::units_per_panel(a->n);
    const size_t braw = m ? 0 : up256(R * n), bunits = m ? 0 : up256(R / 16 * ku * (size_t)pkq8::kUnitBytes);
    if ((e = reserve(l.c, bq + bd + 2 * bw + bo + braw + bunits)))
        return e;
    char *p = l.c->dev;
    int8_t *dq = (int8_t *)p;
    float *dd = (float *)(p + bq);
    float *dws = (float *)(p + bq + bd);
    float *db = (float *)(p + bq + bd + bw);
    float *dout = (float *)(p + bq + bd + 2 * bw);
    hipStream_t s = l.c->stream;
    pk_hip_q8 staged;
    if (!m) {
        int8_t *draw = (int8_t *)(p + bq + bd + 2 * bw + bo);
        staged.hq = w;
        staged.hs = nullptr;
        staged.rows = rows;
        staged.cols = a->n;
        staged.ku = ku;
        staged.w = (int8_t *)(p + bq + bd + 2 * bw + bo + braw);
        staged.s = nullptr;
        if ((e = h2d(l.c, draw, w, R * n, 1, 0)))
            return e;
        if (pkq8::launch_repack(staged.w, draw, rows, a->n, s))
            return launch_fail(-1, "repack launch");
        m = &staged;
    }
    if ((e = h2d(l.c, dq, a->q, T * n, 1, 0)) || (e = h2d(l.c, dd, a->d, T * nb * 4, 1, 0)))
        return e;
    /* the scales a model binds are the uploaded matrix's own, already on the
     * device; other scales are copied */
    const float *wsd = m->s ? m->s + r0 : nullptr;
    if (!m->hs || ws != m->hs + r0) {
        if ((e = h2d(l.c, dws, ws, R * 4, 1, 0)))
            return e;
        wsd = dws;
    }
    if (bias && (e = h2d(l.c, db, bias, R * 4, 1, 0)))
        return e;
    if (add && (e = h2d(l.c, dout, out, R * 4, T, os * 4)))
        return e;
    pk_hip_act da = { dq, dd, a->n, a->qb, a->T };
    /* few frames per row: the split over K, in the lease's own workspace */
    void *skw = nullptr;
    if (a->T <= 16 && a->qb == a->n) {
        if ((e = reserve_split(l.c, pkq8::skinny_workspace_bytes(rows))))
            return e;
        skw = l.c->skw;
    }
    if ((e = launch_product(dout, R, m, r0, rows, wsd, bias ? db : nullptr, &da, add, rmode, s, nullptr, skw)))
        return e;
    return d2h(l.c, out, os * 4, dout, R * 4, T);
}

int pk_hip_quantize_dev(pk_hip_act *a, const float *x, size_t xs, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if ((e = check_act(a, false)))
        return e;
    if (a->T == 0)
        return PK_HIP_OK;
    if (!x || xs < a->n || xs % 4 || ((uintptr_t)x & 15) || ((uintptr_t)a->q & 15))
        return fail(PK_HIP_EINVAL, "quantize_dev: x and q 16-byte aligned, xs >= n and a multiple of 4");
    return launch_quant(a, x, xs, (hipStream_t)stream);
}

int pk_hip_gemm_q8_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                       const float *ws, const float *bias, const pk_hip_act *a, int add, int rmode,
                       void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!m)
        return fail(PK_HIP_ENOTUP, "gemm_q8_dev: no matrix");
    if ((e = check_act(a, true)))
        return e;
    if (a->T == 0)
        return PK_HIP_OK;
    if (!out || !ws)
        return fail(PK_HIP_EINVAL, "gemm_q8_dev: out or ws is NULL");
    if ((uintptr_t)a->q & 15)
        return fail(PK_HIP_EINVAL, "gemm_q8_dev: a->q must be 16-byte aligned");
    if (a->T > 1 && os < rows)
        return fail(PK_HIP_EINVAL, "gemm_q8_dev: output stride %zu is under rows %u", os, rows);
    if (rmode < 0 || rmode > 3)
        return fail(PK_HIP_EROUND, "gemm_q8_dev: rmode %d", rmode);
    if ((e = check_panel(m, r0, rows, a->n)))
        return e;
    return launch_product(out, os, m, r0, rows, ws, bias, a, add, rmode, (hipStream_t)stream);
}

size_t pk_hip_packed_bytes(uint32_t n, uint32_t T) { return (size_t)pkq8::packed_bytes(n, T); }

int pk_hip_quantize_packed_dev(pk_hip_act *a, int8_t *qp, const float *x, size_t xs, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!a)
        return fail(PK_HIP_EINVAL, "quantize_packed_dev: act is NULL");
    if (a->T == 0)
        return PK_HIP_OK;
    if (!a->d || !qp || a->n == 0 || a->n % 32 || a->n > 4096 ||
        !(a->qb == a->n || ((a->qb == 32 || a->qb == 64) && a->n % a->qb == 0)))
        return fail(PK_HIP_EINVAL, "quantize_packed_dev: blocks of the whole row, 32 or 64 inputs, n a "
                                   "multiple of 32 up to 4096, d and qp set");
    if (xs < a->n || xs % 4 || ((uintptr_t)x & 15) || ((uintptr_t)qp & 15) || ((uintptr_t)a->q & 15))
        return fail(PK_HIP_EINVAL, "quantize_packed_dev: x, q and qp 16-byte aligned, xs >= n and a multiple of 4");
    const char *name = "";
    if (const int r = pkq8::launch_quantize_packed(a->q, qp, a->d, x, xs, a->n, a->qb, a->T, (hipStream_t)stream, &name))
        return launch_fail(r, "quantize_packed launch");
    g_kernel = name;
    return PK_HIP_OK;
}

int pk_hip_gemm_q8_packed_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                              const float *ws, const float *bias, const pk_hip_act *a, const int8_t *qp,
                              int add, int rmode, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!m)
        return fail(PK_HIP_ENOTUP, "gemm_q8_packed_dev: no matrix");
    if (!a)
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_dev: act is NULL");
    if (a->T == 0)
        return PK_HIP_OK;
    if (!a->d || !qp || ((uintptr_t)qp & 15) || a->n % 32 || a->n > 16384 ||
        !(a->qb == a->n || ((a->qb == 32 || a->qb == 64) && a->n % a->qb == 0)))
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_dev: blocks of the whole row, 32 or 64 inputs, d and a "
                                   "16-byte aligned qp");
    if (!out || !ws)
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_dev: out or ws is NULL");
    if (a->T > 1 && os < rows)
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_dev: output stride %zu is under rows %u", os, rows);
    if (rmode < 0 || rmode > 3)
        return fail(PK_HIP_EROUND, "gemm_q8_packed_dev: rmode %d", rmode);
    if ((e = check_panel(m, r0, rows, a->n)))
        return e;
    return launch_product(out, os, m, r0, rows, ws, bias, a, add, rmode, (hipStream_t)stream, qp);
}

static int check_work(const void *work, size_t work_bytes, uint32_t rows, const char *who) {
    if (!work)
        return PK_HIP_OK;
    if ((uintptr_t)work & 255)
        return fail(PK_HIP_EINVAL, "%s: the workspace must be 256-byte aligned", who);
    const size_t need = pkq8::skinny_workspace_bytes(rows);
    if (work_bytes < need)
        return fail(PK_HIP_EINVAL, "%s: workspace of %zu bytes, %zu needed for %u rows", who, work_bytes, need, rows);
    return PK_HIP_OK;
}

int pk_hip_gemm_q8_ws_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                          const float *ws, const float *bias, const pk_hip_act *a, int add, int rmode,
                          void *work, size_t work_bytes, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!m)
        return fail(PK_HIP_ENOTUP, "gemm_q8_ws_dev: no matrix");
    if ((e = check_act(a, true)))
        return e;
    if (a->T == 0)
        return PK_HIP_OK;
    if (!out || !ws)
        return fail(PK_HIP_EINVAL, "gemm_q8_ws_dev: out or ws is NULL");
    if ((uintptr_t)a->q & 15)
        return fail(PK_HIP_EINVAL, "gemm_q8_ws_dev: a->q must be 16-byte aligned");
    if (a->T > 1 && os < rows)
        return fail(PK_HIP_EINVAL, "gemm_q8_ws_dev: output stride %zu is under rows %u", os, rows);
    if (rmode < 0 || rmode > 3)
        return fail(PK_HIP_EROUND, "gemm_q8_ws_dev: rmode %d", rmode);
    if ((e = check_panel(m, r0, rows, a->n)) || (e = check_work(work, work_bytes, rows, "gemm_q8_ws_dev")))
        return e;
    return launch_product(out, os, m, r0, rows, ws, bias, a, add, rmode, (hipStream_t)stream, nullptr, work);
}

int pk_hip_gemm_q8_packed_ws_dev(float *out, size_t os, const pk_hip_q8 *m, uint32_t r0, uint32_t rows,
                                 const float *ws, const float *bias, const pk_hip_act *a, const int8_t *qp,
                                 int add, int rmode, void *work, size_t work_bytes, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!m)
        return fail(PK_HIP_ENOTUP, "gemm_q8_packed_ws_dev: no matrix");
    if (!a)
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_ws_dev: act is NULL");
    if (a->T == 0)
        return PK_HIP_OK;
    if (!a->d || !qp || ((uintptr_t)qp & 15) || a->n % 32 || a->n > 16384 ||
        !(a->qb == a->n || ((a->qb == 32 || a->qb == 64) && a->n % a->qb == 0)))
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_ws_dev: blocks of the whole row, 32 or 64 inputs, d and a "
                                   "16-byte aligned qp");
    if (!out || !ws)
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_ws_dev: out or ws is NULL");
    if (a->T > 1 && os < rows)
        return fail(PK_HIP_EINVAL, "gemm_q8_packed_ws_dev: output stride %zu is under rows %u", os, rows);
    if (rmode < 0 || rmode > 3)
        return fail(PK_HIP_EROUND, "gemm_q8_packed_ws_dev: rmode %d", rmode);
    if ((e = check_panel(m, r0, rows, a->n)) || (e = check_work(work, work_bytes, rows, "gemm_q8_packed_ws_dev")))
        return e;
    return launch_product(out, os, m, r0, rows, ws, bias, a, add, rmode, (hipStream_t)stream, qp, work);
}

int pk_hip_gemm_q8_batch_dev(const pk_hip_job *jobs, uint32_t njobs, int rmode, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!jobs || njobs == 0 || njobs > (uint32_t)pkq8::kMaxJobs)
        return fail(PK_HIP_EINVAL, "gemm_q8_batch_dev: njobs %u is not in [1, %d]", njobs, pkq8::kMaxJobs);
    if (rmode < 0 || rmode > 3)
        return fail(PK_HIP_EROUND, "gemm_q8_batch_dev: rmode %d", rmode);
    pkq8::JobTable tab;
    tab.njobs = njobs;
    const uint32_t n = jobs[0].a.n, qb = jobs[0].a.qb;
    for (uint32_t j = 0; j < njobs; j++) {
        const pk_hip_job &jb = jobs[j];
        const pk_hip_act *a = &jb.a;
        if (!jb.m)
            return fail(PK_HIP_ENOTUP, "gemm_q8_batch_dev: job %u has no matrix", j);
        if (a->n != n || a->qb != qb || !(qb == n || qb == 32 || qb == 64) || n % qb || n % 32 || n > 16384)
            return fail(PK_HIP_EINVAL,
                        "gemm_q8_batch_dev: job %u has n %u qb %u; the jobs share n and qb (n, 32 or 64)", j,
                        a->n, a->qb);
        if (a->T && (!a->d || !jb.qp || ((uintptr_t)jb.qp & 15) || !jb.out || !jb.ws))
            return fail(PK_HIP_EINVAL, "gemm_q8_batch_dev: job %u needs out, ws, d and a 16-byte aligned qp", j);
        if (a->T > 1 && jb.os < jb.rows)
            return fail(PK_HIP_EINVAL, "gemm_q8_batch_dev: job %u output stride %zu is under rows %u", j, jb.os,
                        jb.rows);
        if ((e = check_panel(jb.m, jb.r0, jb.rows, n)))
            return e;
        if (jb.m->ku != jobs[0].m->ku)
            return fail(PK_HIP_EINVAL, "gemm_q8_batch_dev: job %u's matrix is padded to other units", j);
        pkq8::GemmArgs &g = tab.g[j];
        g.w = jb.m->w + (size_t)(jb.r0 / 16) * pkq8::kUnitBytes;
        g.wstride = (uint64_t)(jb.m->rows / 16) * pkq8::kUnitBytes;
        g.ws = jb.ws;
        g.bias = jb.bias;
        g.rows = jb.rows;
        g.n = n;
        g.ku = jb.m->ku;
        g.kr = pkq8::units_with_data(jb.m->cols);
        g.qb = qb;
        g.nb = n / qb;
        g.add = jb.add;
        g.rmode = rmode;
        tab.s[j] = pkq8::Seg{ jb.out, jb.qp, a->d, (uint64_t)jb.os,
                              (uint64_t)pkq8::packed_groups(a->T) * pkq8::kUnitBytes, a->T, 0 };
    }
    const char *name = "";
    if (const int r = pkq8::launch_gemm_batch(tab, (hipStream_t)stream, &name))
        return launch_fail(r, "gemm_q8_batch_dev launch");
    g_kernel = name;
    return PK_HIP_OK;
}

int pk_hip_gemm_q8_grouped_dev(const pk_hip_q8 *m, uint32_t r0, uint32_t rows, const float *ws,
                               const float *bias, const pk_hip_seg *segs, uint32_t nseg, int add,
                               void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!m)
        return fail(PK_HIP_ENOTUP, "gemm_q8_grouped_dev: no matrix");
    if (!segs || nseg == 0 || nseg > (uint32_t)pkq8::kMaxSegs)
        return fail(PK_HIP_EINVAL, "gemm_q8_grouped_dev: nseg %u is not in [1, %d]", nseg, pkq8::kMaxSegs);
    if (!ws)
        return fail(PK_HIP_EINVAL, "gemm_q8_grouped_dev: ws is NULL");
    const uint32_t n = segs[0].a.n, qb = segs[0].a.qb;
    pkq8::SegTable tab;
    tab.nseg = 0;
    for (uint32_t i = 0; i < nseg; i++) {
        const pk_hip_seg &sg = segs[i];
        if ((e = check_act(&sg.a, true)))
            return e;
        if (sg.a.T == 0)
            continue;
        if (sg.a.n != n || sg.a.qb != qb)
            return fail(PK_HIP_EINVAL, "gemm_q8_grouped_dev: segment %u has n %u qb %u, not %u %u", i,
                        sg.a.n, sg.a.qb, n, qb);
        if (!sg.out || ((uintptr_t)sg.a.q & 15) || (sg.a.T > 1 && sg.os < rows))
            return fail(PK_HIP_EINVAL, "gemm_q8_grouped_dev: segment %u: out NULL, q unaligned or os < rows", i);
        tab.s[tab.nseg++] = pkq8::Seg{ sg.out, sg.a.q, sg.a.d, (uint64_t)sg.os, 0, sg.a.T, 0 };
    }
    if (tab.nseg == 0)
        return PK_HIP_OK;
    if ((e = check_panel(m, r0, rows, n)))
        return e;
    pkq8::GemmArgs g;
    g.w = m->w + (size_t)(r0 / 16) * pkq8::kUnitBytes;
    g.wstride = (uint64_t)(m->rows / 16) * pkq8::kUnitBytes;
    g.ws = ws;
    g.bias = bias;
    g.rows = rows;
    g.n = n;
    g.ku = m->ku;
    g.kr = pkq8::units_with_data(m->cols);
    g.qb = qb;
    g.nb = n / qb;
    g.add = add;
    g.rmode = 0;
    const char *name = "";
    if (const int r = pkq8::launch_gemm(g, tab, (hipStream_t)stream, &name))
        return launch_fail(r, "gemm_q8_grouped launch");
    g_kernel = name;
    return PK_HIP_OK;
}

}  // extern "C"

/* ----------------------------------------- the device-resident layer --- */

namespace {

bool al16(const void *p) { return p && ((uintptr_t)p & 15) == 0; }

bool blocks_ok(const pk_hip_act *a, bool whole) {
    return ((a->qb == 32 || a->qb == 64) && a->n % a->qb == 0) || (whole && a->qb == a->n);
}

#define PK_LAUNCH(call, what)                                            \
    do {                                                                 \
        if (const int r_ = (call))                                       \
            return launch_fail(r_, what);                                \
    } while (0)

/* The layer's workspace, carved in 256-byte aligned pieces; with base NULL
 * only the size. */
struct LayerWs {
    int8_t *act_qp, *hid_qp;
    float *act_d, *hid_d, *u, *qf, *kf, *vf, *pf, *S, *of;
};

size_t layer_carve(LayerWs *w, char *base, const pk_hip_layer *L, uint32_t T, uint32_t qb) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char *p = base ? base + off : nullptr;
        off += (bytes + 255) & ~(size_t)255;
        return p;
    };
    const size_t D = L->D, F = L->F, R = 2 * (size_t)T - 1, U = F > 2 * D ? F : 2 * D;
    w->act_qp = (int8_t *)take(pkq8::packed_bytes(L->D, T));
    w->act_d = (float *)take(T * (D / qb) * 4);
    w->hid_qp = (int8_t *)take(pkq8::packed_bytes(L->F, T));
    w->hid_d = (float *)take(T * (F / qb) * 4);
    w->u = (float *)take(T * U * 4);
    w->qf = (float *)take(T * D * 4);
    w->kf = (float *)take(T * D * 4);
    w->vf = (float *)take(T * D * 4);
    w->pf = (float *)take(R * D * 4);
    w->S = (float *)take(pkq8::att_workspace_floats(T, L->H) * 4);
    w->of = (float *)take(T * D * 4);
    return off;
}

bool mat_is(const pk_hip_q8 *m, uint32_t rows, uint32_t cols) { return m && m->rows == rows && m->cols == cols; }

int layer_check(const pk_hip_layer *L, uint32_t qb) {
    if (!L)
        return fail(PK_HIP_EINVAL, "layer_dev: no layer");
    const uint32_t D = L->D, F = L->F, H = L->H;
    if (D == 0 || D % 64 || D > 4096 || F == 0 || F % 64 || F > 4096 || H == 0 || D % H || (D / H) % 16 ||
        L->K == 0 || L->K > 33 || !(qb == 32 || qb == 64) || !(L->eps >= 0.0f))
        return fail(PK_HIP_EINVAL, "layer_dev: D and F multiples of 64 up to 4096, heads of a multiple of 16, "
                                   "1 to 33 taps, blocks of 32 or 64");
    const float *v[] = { L->ff1_nw, L->ff1_nb, L->att_nw, L->att_nb, L->conv_nw, L->conv_nb, L->ff2_nw,
                         L->ff2_nb, L->out_nw, L->out_nb, L->bias_u, L->bias_v, L->dw_b };
    for (const float *p : v)
        if (!al16(p))
            return fail(PK_HIP_EINVAL, "layer_dev: a vector is NULL or not 16-byte aligned");
    if (!L->dw)
        return fail(PK_HIP_EINVAL, "layer_dev: dw is NULL");
    if (!mat_is(L->ff1_up, F, D) || !mat_is(L->ff2_up, F, D) || !mat_is(L->ff1_down, D, F) ||
        !mat_is(L->ff2_down, D, F) || !mat_is(L->q, D, D) || !mat_is(L->k, D, D) || !mat_is(L->v, D, D) ||
        !mat_is(L->pos, D, D) || !mat_is(L->o, D, D) || !mat_is(L->pw1, 2 * D, D) || !mat_is(L->pw2, D, D))
        return fail(PK_HIP_ENOTUP, "layer_dev: a matrix is missing or of the wrong shape");
    return PK_HIP_OK;
}

}  // namespace

extern "C" {

int pk_hip_normq_dev(pk_hip_act *a, int8_t *qp, const float *x, const float *w, const float *b, float eps,
                     void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!a)
        return fail(PK_HIP_EINVAL, "normq_dev: act is NULL");
    if (a->T == 0)
        return PK_HIP_OK;
    if (!a->d || !al16(qp) || !al16(x) || !al16(w) || !al16(b) || a->n == 0 || a->n % 64 || a->n > 4096 ||
        !blocks_ok(a, true))
        return fail(PK_HIP_EINVAL, "normq_dev: n a multiple of 64 up to 4096 in blocks of the whole row, 32 or "
                                   "64; d set, qp, x, w and b 16-byte aligned");
    PK_LAUNCH(pkq8::launch_normq(qp, a->d, x, a->n, a->T, w, b, eps, a->qb, (hipStream_t)stream), "normq launch");
    g_kernel = "normq";
    return PK_HIP_OK;
}

int pk_hip_siluq_dev(pk_hip_act *a, int8_t *qp, const float *x, size_t xs, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!a)
        return fail(PK_HIP_EINVAL, "siluq_dev: act is NULL");
    if (a->T == 0)
        return PK_HIP_OK;
    if (!a->d || !al16(qp) || !al16(x) || a->n == 0 || a->n % 32 || a->n > 4096 || !blocks_ok(a, true) ||
        xs < a->n || xs % 4)
        return fail(PK_HIP_EINVAL, "siluq_dev: n a multiple of 32 up to 4096 in blocks of the whole row, 32 or "
                                   "64; d set, qp and x 16-byte aligned, xs >= n and a multiple of 4");
    const char *name = "";
    PK_LAUNCH(pkq8::launch_quantize_packed(nullptr, qp, a->d, x, xs, a->n, a->qb, a->T, (hipStream_t)stream,
                                           &name, pkq8::kOpSilu),
              "siluq launch");
    g_kernel = name;
    return PK_HIP_OK;
}

int pk_hip_dwq_dev(pk_hip_act *a, int8_t *qp, const float *u, const float *w, const float *b, uint32_t K,
                   void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!a)
        return fail(PK_HIP_EINVAL, "dwq_dev: act is NULL");
    if (a->T == 0)
        return PK_HIP_OK;
    if (!a->d || !al16(qp) || !u || !w || !b || a->n == 0 || a->n % 64 || !blocks_ok(a, false) || K == 0 ||
        K > 33)
        return fail(PK_HIP_EINVAL, "dwq_dev: n a multiple of 64 in blocks of 32 or 64, 1 to 33 taps; d, u, w, b "
                                   "set and qp 16-byte aligned");
    PK_LAUNCH(pkq8::launch_dwq(qp, a->d, u, a->T, a->n, w, b, K, a->qb, (hipStream_t)stream), "dwq launch");
    g_kernel = "dwq";
    return PK_HIP_OK;
}

int pk_hip_layernorm_dev(float *x, uint32_t T, uint32_t n, const float *w, const float *b, float eps,
                         void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (T == 0)
        return PK_HIP_OK;
    if (!al16(x) || !al16(w) || !al16(b) || n == 0 || n % 64 || n > 4096)
        return fail(PK_HIP_EINVAL, "layernorm_dev: n a multiple of 64 up to 4096; x, w, b 16-byte aligned");
    PK_LAUNCH(pkq8::launch_norm(x, n, T, w, b, eps, (hipStream_t)stream), "layernorm launch");
    g_kernel = "norm";
    return PK_HIP_OK;
}

size_t pk_hip_attention_workspace(uint32_t T, uint32_t H) {
    return pkq8::att_workspace_floats(T, H) * sizeof(float);
}

int pk_hip_attention_dev(float *o, const float *q, const float *k, const float *v, const float *p,
                         const float *bias_u, const float *bias_v, uint32_t T, uint32_t D, uint32_t H, void *ws,
                         size_t ws_bytes, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (T == 0)
        return PK_HIP_OK;
    if (!o || !q || !k || !v || !p || !bias_u || !bias_v || !ws || H == 0 || D % H || (D / H) % 16)
        return fail(PK_HIP_EINVAL, "attention_dev: heads of a multiple of 16 dimensions, every pointer set");
    if (ws_bytes < pk_hip_attention_workspace(T, H))
        return fail(PK_HIP_EINVAL, "attention_dev: workspace of %zu bytes, %zu needed", ws_bytes,
                    pk_hip_attention_workspace(T, H));
    PK_LAUNCH(pkq8::launch_attention(o, (float *)ws, q, k, v, p, bias_u, bias_v, T, D, H, (hipStream_t)stream),
              "attention launch");
    g_kernel = "attention";
    return PK_HIP_OK;
}

int pk_hip_attention_noalloc_dev(float *o, const float *q, const float *k, const float *v, const float *p,
                                 const float *bias_u, const float *bias_v, uint32_t T, uint32_t D, uint32_t H,
                                 void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (T == 0)
        return PK_HIP_OK;
    if (!o || !q || !k || !v || !p || !bias_u || !bias_v || H == 0 || D % H || (D / H) % 16)
        return fail(PK_HIP_EINVAL, "attention_noalloc_dev: heads of a multiple of 16 dimensions, every pointer set");
    const size_t need = pk_hip_attention_workspace(T, H);
    if (need > pkq8::kStaticScratchBytes)
        return fail(PK_HIP_EINVAL,
                    "attention_noalloc_dev: %u frames of %u heads need %zu bytes of scores, over the static "
                    "scratch's %zu", T, H, need, pkq8::kStaticScratchBytes);
    int dev = -1;
    PK_TRY(hipGetDevice(&dev));
    int se = 0;
    hipEvent_t last = nullptr;
    void *ws = pkq8::static_scratch(dev, &se, &last);
    if (!ws)
        return hip_fail((hipError_t)se, "attention_noalloc_dev: the static scratch's address");
    /* Calls on one GPU share the scratch: outside stream capture each call
     * waits on its stream for the last one to finish with it (an event of
     * the device, recorded after every call; the lock keeps wait, launch and
     * record of two host threads from interleaving). A captured call records
     * neither (a captured wait on an event recorded outside the capture is
     * not allowed): the graph's own order, and the caller's between replays
     * and other calls, keep its uses apart. */
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    PK_TRY(hipStreamIsCapturing((hipStream_t)stream, &cs));
    static std::mutex mu;
    std::lock_guard<std::mutex> lk(mu);
    if (cs == hipStreamCaptureStatusNone)
        PK_TRY(hipStreamWaitEvent((hipStream_t)stream, last, 0));
    PK_LAUNCH(pkq8::launch_attention(o, (float *)ws, q, k, v, p, bias_u, bias_v, T, D, H, (hipStream_t)stream),
              "attention launch");
    if (cs == hipStreamCaptureStatusNone)
        PK_TRY(hipEventRecord(last, (hipStream_t)stream));
    g_kernel = "attention";
    return PK_HIP_OK;
}

size_t pk_hip_layer_workspace(const pk_hip_layer *L, uint32_t T, uint32_t qb) {
    if (!L || T == 0 || !(qb == 32 || qb == 64))
        return 0;
    LayerWs w;
    return layer_carve(&w, nullptr, L, T, qb);
}

int pk_hip_layer_dev(const pk_hip_layer *L, float *x, uint32_t T, const int8_t *ape_qp, const float *ape_d,
                     uint32_t qb, void *ws, size_t ws_bytes, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if ((e = layer_check(L, qb)))
        return e;
    if (T == 0)
        return PK_HIP_OK;
    if (!al16(x) || !al16(ape_qp) || !ape_d || !al16(ws))
        return fail(PK_HIP_EINVAL, "layer_dev: x, ape_qp and ws 16-byte aligned, ape_d set");
    LayerWs w;
    const size_t need = layer_carve(&w, (char *)ws, L, T, qb);
    if (ws_bytes < need)
        return fail(PK_HIP_EINVAL, "layer_dev: workspace of %zu bytes, %zu needed", ws_bytes, need);
    hipStream_t s = (hipStream_t)stream;
    const uint32_t D = L->D, F = L->F, R = 2 * T - 1;
    pk_hip_act act = { nullptr, w.act_d, D, qb, T }, hid = { nullptr, w.hid_d, F, qb, T };
    pk_hip_act ape = { nullptr, const_cast<float *>(ape_d), D, qb, R };
    const char *name = "";
    auto gemm = [&](float *out, size_t os, const pk_hip_q8 *m, const pk_hip_act *a, const int8_t *qp, int add) {
        return launch_product(out, os, m, 0, m->rows, m->s, nullptr, a, add, 0, s, qp);
    };
    /* ff (core/encoder.c:321-327): x += down(siluq(up(normq(x)))); the SiLU
     * quantize in the up product's epilogue where its tile has one (the
     * same bytes and scales: the fp32 hidden activations are never written),
     * else a pass of its own over them */
    auto ff = [&](const float *nw, const float *nb, const pk_hip_q8 *up, const pk_hip_q8 *down) {
        PK_LAUNCH(pkq8::launch_normq(w.act_qp, w.act_d, x, D, T, nw, nb, L->eps, qb, s), "layer normq launch");
        const int f = launch_product_siluq(up, &act, w.act_qp, w.hid_qp, w.hid_d, qb, s);
        if (f > 0) {
            int r = gemm(w.u, F, up, &act, w.act_qp, 0);
            if (r)
                return r;
            PK_LAUNCH(pkq8::launch_quantize_packed(nullptr, w.hid_qp, w.hid_d, w.u, F, F, qb, T, s, &name,
                                                   pkq8::kOpSilu),
                      "layer siluq launch");
        } else if (f < 0) {
            return -f;
        }
        return gemm(x, D, down, &hid, w.hid_qp, 1);
    };
    if ((e = ff(L->ff1_nw, L->ff1_nb, L->ff1_up, L->ff1_down)))
        return e;
    /* the attention (core/encoder.c:339-352) */
    PK_LAUNCH(pkq8::launch_normq(w.act_qp, w.act_d, x, D, T, L->att_nw, L->att_nb, L->eps, qb, s),
              "layer normq launch");
    {
        /* q, k and v of one activation and the positions' projection: one
         * launch (independent products, each its bits alone) */
        const pk_hip_job jobs[4] = {
            { w.qf, D, L->q, 0, D, L->q->s, nullptr, act, w.act_qp, 0 },
            { w.kf, D, L->k, 0, D, L->k->s, nullptr, act, w.act_qp, 0 },
            { w.vf, D, L->v, 0, D, L->v->s, nullptr, act, w.act_qp, 0 },
            { w.pf, D, L->pos, 0, D, L->pos->s, nullptr, ape, ape_qp, 0 },
        };
        if ((e = pk_hip_gemm_q8_batch_dev(jobs, 4, 0, stream)))
            return e;
    }
    /* the attention's output quantized in the PV's epilogue; where that
     * kernel has no such epilogue (the VALU chains), written and quantized
     * by a pass of its own */
    const int ra = pkq8::launch_attention(w.of, w.S, w.qf, w.kf, w.vf, w.pf, L->bias_u, L->bias_v, T, D, L->H, s,
                                          w.act_qp, w.act_d, qb);
    if (ra == -2) {
        PK_LAUNCH(pkq8::launch_attention(w.of, w.S, w.qf, w.kf, w.vf, w.pf, L->bias_u, L->bias_v, T, D, L->H, s),
                  "layer attention launch");
        PK_LAUNCH(pkq8::launch_quantize_packed(nullptr, w.act_qp, w.act_d, w.of, D, D, qb, T, s, &name),
                  "layer quantize launch");
    } else if (ra) {
        return launch_fail(ra, "layer attention launch");
    }
    if ((e = gemm(x, D, L->o, &act, w.act_qp, 1)))
        return e;
    /* the convolution module (core/encoder.c:354-362) */
    PK_LAUNCH(pkq8::launch_normq(w.act_qp, w.act_d, x, D, T, L->conv_nw, L->conv_nb, L->eps, qb, s),
              "layer normq launch");
    if ((e = gemm(w.u, 2 * D, L->pw1, &act, w.act_qp, 0)))
        return e;
    PK_LAUNCH(pkq8::launch_dwq(w.act_qp, w.act_d, w.u, T, D, L->dw, L->dw_b, L->K, qb, s), "layer dwq launch");
    if ((e = gemm(x, D, L->pw2, &act, w.act_qp, 1)))
        return e;
    if ((e = ff(L->ff2_nw, L->ff2_nb, L->ff2_up, L->ff2_down)))
        return e;
    PK_LAUNCH(pkq8::launch_norm(x, D, T, L->out_nw, L->out_nb, L->eps, s), "layer norm launch");
    g_kernel = "layer";
    return PK_HIP_OK;
}

/* ------------------------------------------ the decoder's token steps --- */

int pk_hip_gemv_dev(float *out, const pk_hip_q8 *m, const float *bias, const float *x, int add, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!m)
        return fail(PK_HIP_ENOTUP, "gemv_dev: no matrix");
    if (!out || !x || m->cols > 4096)
        return fail(PK_HIP_EINVAL, "gemv_dev: out and x set, cols <= 4096");
    PK_LAUNCH(pkq8::launch_gemv(out, m->w, (uint64_t)(m->rows / 16) * pkq8::kUnitBytes, m->s, bias, x, m->rows,
                                m->cols, pkq8::units_with_data(m->cols), add, (hipStream_t)stream),
              "gemv launch");
    g_kernel = "gemv";
    return PK_HIP_OK;
}

int pk_hip_lstm_step_dev(float *h_out, float *c, const float *h_in, const float *x, const pk_hip_q8 *wx,
                         const pk_hip_q8 *wh, const float *b, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!wx || !wh)
        return fail(PK_HIP_ENOTUP, "lstm_step_dev: no matrix");
    const uint32_t P = wx->cols;
    if (wx->rows != 4 * P || wh->rows != 4 * P || wh->cols != P || P % 16 || P > 4096)
        return fail(PK_HIP_EINVAL, "lstm_step_dev: wx and wh [4P][P], P a multiple of 16 up to 4096");
    if (!h_out || !c || !h_in || !x || !b || h_out == h_in)
        return fail(PK_HIP_EINVAL, "lstm_step_dev: every pointer set, h_out not h_in");
    PK_LAUNCH(pkq8::launch_lstm(h_out, c, h_in, x, wx->w, wx->s, wh->w, wh->s,
                                (uint64_t)(wx->rows / 16) * pkq8::kUnitBytes, b, P, pkq8::units_with_data(P),
                                (hipStream_t)stream),
              "lstm launch");
    g_kernel = "lstm";
    return PK_HIP_OK;
}

int pk_hip_joint_dev(float *logit, uint32_t *tok_dur, const pk_hip_q8 *jout, const float *jout_b, const float *f,
                     const float *gp, uint32_t V, uint32_t n_dur, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!jout)
        return fail(PK_HIP_ENOTUP, "joint_dev: no matrix");
    if (!logit || !tok_dur || !f || !gp || jout->cols > 4096 || n_dur == 0 || V + 1 + n_dur > jout->rows)
        return fail(PK_HIP_EINVAL, "joint_dev: every pointer set, cols <= 4096, V + 1 + n_dur <= rows");
    PK_LAUNCH(pkq8::launch_joint(logit, tok_dur, jout->w, (uint64_t)(jout->rows / 16) * pkq8::kUnitBytes, jout->s,
                                 jout_b, f, gp, jout->rows, jout->cols, pkq8::units_with_data(jout->cols), V, n_dur,
                                 (hipStream_t)stream),
              "joint launch");
    g_kernel = "joint";
    return PK_HIP_OK;
}

static int search_shape(const pk_hip_decoder *d) {
    if (!d || !d->embed || !d->jpred || !d->jout || d->L == 0 || d->L > PK_HIP_DEC_MAX_LAYERS || d->n_dur == 0 ||
        d->n_dur > 64 || d->P == 0 || d->P % 16 || d->P > 1024 || d->J == 0 || d->J % 16 || d->J > 1024 ||
        d->V + 1 > 2048 || d->blank > d->V || d->max_symbols == 0)
        return fail(PK_HIP_EINVAL, "search: P and J multiples of 16 up to 1024, 1 <= L <= %d, 1 <= n_dur <= 64, "
                                   "V + 1 <= 2048, blank <= V, max_symbols >= 1, embed, jpred and jout set",
                    PK_HIP_DEC_MAX_LAYERS);
    for (uint32_t l = 0; l < d->L; l++) {
        const pk_hip_q8 *x = d->wx[l], *h = d->wh[l];
        if (!x || !h || x->rows != 4 * d->P || x->cols != d->P || h->rows != 4 * d->P || h->cols != d->P)
            return fail(PK_HIP_EINVAL, "search: layer %u's wx and wh must be uploaded [4P][P] matrices", l);
    }
    if (d->jpred->rows != d->J || d->jpred->cols != d->P || d->jout->cols != d->J ||
        d->V + 1 + d->n_dur > d->jout->rows)
        return fail(PK_HIP_EINVAL, "search: jpred [J][P], jout [rows][J] with rows >= V + 1 + n_dur");
    return PK_HIP_OK;
}

size_t pk_hip_search_workspace(const pk_hip_decoder *d, uint32_t cap) {
    if (search_shape(d))
        return 0;
    return pkq8::search_workspace_bytes(d->L, d->P, d->J, d->jout->rows, cap);
}

int pk_hip_search_dev(const pk_hip_decoder *d, const float *f, uint32_t T, int32_t *toks, uint32_t cap,
                      uint32_t *ntoks, void *ws, size_t ws_bytes, uint32_t spin_limit, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if ((e = search_shape(d)))
        return e;
    if (!ntoks || (T && (!f || !toks)))
        return fail(PK_HIP_EINVAL, "search: f, toks and ntoks set");
    *ntoks = 0;
    if (T == 0)
        return PK_HIP_OK;
    if ((uint64_t)cap < (uint64_t)T * d->max_symbols)
        return fail(PK_HIP_EINVAL, "search: cap %u is under T * max_symbols = %llu", cap,
                    (unsigned long long)T * d->max_symbols);
    const size_t need = pkq8::search_workspace_bytes(d->L, d->P, d->J, d->jout->rows, cap);
    if (!ws || ((uintptr_t)ws & 255) || ws_bytes < need)
        return fail(PK_HIP_EINVAL, "search: a 256-byte aligned workspace of %zu bytes (%zu given)", need, ws_bytes);
    pkq8::SearchArgs a{};
    a.f = f;
    a.embed = d->embed;
    for (uint32_t l = 0; l < d->L; l++) {
        a.wx[l] = d->wx[l]->w;
        a.wh[l] = d->wh[l]->w;
        a.wxs[l] = d->wx[l]->s;
        a.whs[l] = d->wh[l]->s;
        a.b[l] = d->b[l];
    }
    a.jpred = d->jpred->w;
    a.jout = d->jout->w;
    a.jpred_s = d->jpred->s;
    a.jout_s = d->jout->s;
    a.jpred_b = d->jpred_b;
    a.jout_b = d->jout_b;
    a.lstm_stride = (uint64_t)(4 * d->P / 16) * pkq8::kUnitBytes;
    a.jpred_stride = (uint64_t)(d->J / 16) * pkq8::kUnitBytes;
    a.jout_stride = (uint64_t)(d->jout->rows / 16) * pkq8::kUnitBytes;
    a.P = d->P;
    a.L = d->L;
    a.J = d->J;
    a.V = d->V;
    a.n_dur = d->n_dur;
    a.rows_out = d->jout->rows;
    a.blank = d->blank;
    a.max_symbols = d->max_symbols;
    a.T = T;
    a.cap = cap;
    a.kr_p = pkq8::units_with_data(d->P);
    a.kr_j = pkq8::units_with_data(d->J);
    a.spin = spin_limit ? spin_limit : 1u << 22;
    for (uint32_t i = 0; i < d->n_dur; i++)
        a.dur[i] = d->dur[i];
    hipStream_t s = (hipStream_t)stream;
    PK_LAUNCH(pkq8::launch_search(a, ws, s), "search launch");
    g_kernel = "search";
    uint32_t res[2] = { 0, 0 }, flag[2] = { 0, 0 };
    PK_TRY(hipMemcpyAsync(res, a.out, sizeof res, hipMemcpyDeviceToHost, s));
    PK_TRY(hipMemcpyAsync(flag, a.sync, sizeof flag, hipMemcpyDeviceToHost, s));
    PK_TRY(hipStreamSynchronize(s));
    if (flag[1])
        return fail(PK_HIP_ETIMEOUT, "search: a grid-wide wait ran past its %u iterations; the launch left early",
                    a.spin);
    if (res[1] == 2 || res[0] > cap)
        return fail(PK_HIP_EINVAL, "search: more than cap %u tokens", cap);
    if (res[0])
        PK_TRY(hipMemcpy(toks, a.toks, (size_t)res[0] * 12, hipMemcpyDeviceToHost));
    *ntoks = res[0];
    return PK_HIP_OK;
}

int pk_hip_empty_dev(void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    PK_LAUNCH(pkq8::launch_empty((hipStream_t)stream), "empty launch");
    g_kernel = "empty";
    return PK_HIP_OK;
}

int pk_hip_stream_read_dev(const void *p, size_t bytes, uint32_t *sink, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (bytes == 0)
        return PK_HIP_OK;
    if (!p || !sink || bytes % 16 || (uintptr_t)p % 16)
        return fail(PK_HIP_EINVAL, "stream_read_dev: p and sink set, p 16-byte aligned, bytes a multiple of 16");
    PK_LAUNCH(pkq8::launch_stream_read(p, bytes, sink, (hipStream_t)stream), "stream read launch");
    g_kernel = "stream_read";
    return PK_HIP_OK;
}

int pk_hip_mfma_rate_dev(uint32_t workgroups, uint32_t iters, uint32_t *sink, void *stream) {
    int e = pk_hip_init();
    if (e)
        return e;
    if (!sink)
        return fail(PK_HIP_EINVAL, "mfma_rate_dev: sink is NULL");
    PK_LAUNCH(pkq8::launch_mfma_rate(workgroups, iters, sink, (hipStream_t)stream), "mfma rate launch");
    g_kernel = "mfma_rate";
    return PK_HIP_OK;
}

}  // extern "C"
