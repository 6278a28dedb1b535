// capi.cpp -- the C ABI of include/gemmkit_hip.h: validation, degenerate cases,
// orientation, route choice and launches.
//
// Layering follows gemmkit's own (ARCHITECTURE.md "The Layer Stack"):
//   checked entries  -> validate_gemm_views and friends (src/api.rs:188-314,
//                       src/adapter.rs:130-273, src/api/batched.rs:31-163),
//                       same conditions, same "gemmkit: ..." wording;
//   unchecked entries-> straight to the dispatch layer (src/api.rs:469-580);
//   dispatch         -> m|n == 0 returns, k == 0 / alpha == 0 scales C
//                       (src/dispatch.rs:345-358, src/dispatch/int.rs:131-163),
//                       orientation swap (src/dispatch.rs:395-417), then the
//                       GEMV route for skinny products or the MFMA tile grid.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include <sys/syscall.h>
#include <unistd.h>

#include "../../include/gemmkit_hip.h"
#include "internal.h"

using namespace gk;

// ------------------------------------------------------------------ state

namespace {

thread_local std::string tl_error;
thread_local hipStream_t tl_stream = nullptr;
thread_local int tl_sync = 1;

// The workspace a call has taken (its event and recorded flag): the call's
// end, or its failure after launching something, records the event on the
// launch stream, which orders the arena's next user on another stream.
thread_local hipEvent_t tl_ws_event = nullptr;
thread_local bool *tl_ws_recorded = nullptr;

void ws_mark_done() {
    if (!tl_ws_recorded) return;
    if (hipEventRecord(tl_ws_event, tl_stream) == hipSuccess) *tl_ws_recorded = true;
    tl_ws_recorded = nullptr;
}

int fail(int code, const char *fmt, ...) {
    ws_mark_done();
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    tl_error = buf;
    return code;
}

int ok() {
    tl_error.clear();
    return GK_OK;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(GK_ERR_DEVICE, "gemmkit: HIP error in %s: %s", what, hipGetErrorString(e));
}

std::once_flag g_init_once;
int g_init_status = GK_OK;
std::string g_init_error;
int g_num_cus = 256;

// ---------------------------------------------------- no-allocation scratch

// Device scratch of gk_gemm_i8_unchecked_noalloc: packed operands and split-K
// partial sums of calls that must not allocate.  Each device holds its own
// copy from module load to process exit.  In host code `scratch` names a
// host-side stand-in, not device memory: kernels get the per-device address
// that hipGetSymbolAddress returns (g_scratch_dev), never the array's name.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_dev[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device with
// that device current.
int scratch_for_current_device(uint8_t **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return fail(GK_ERR_DEVICE, "gemmkit: device %d is beyond the %d devices the no-allocation "
                                   "scratch tracks", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        g_scratch_dev[dev] = (uint8_t *)p;
    }
    *out = g_scratch_dev[dev];
    return GK_OK;
}

int device_init() {
    std::call_once(g_init_once, [] {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n == 0) {
            g_init_status = GK_ERR_DEVICE;
            g_init_error = std::string("gemmkit: no HIP device available (") +
                           hipGetErrorString(e) + ")";
            return;
        }
        int dev = 0;
        (void)hipGetDevice(&dev);
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
            g_num_cus = prop.multiProcessorCount;
        // Set-up of the no-allocation scratch for the initial device (other
        // devices look theirs up on first use); a failure here surfaces in
        // the entry point that needs it.
        uint8_t *sp = nullptr;
        std::string keep = tl_error;
        (void)scratch_for_current_device(&sp);
        tl_error = keep;
    });
    if (g_init_status != GK_OK) return fail(g_init_status, "%s", g_init_error.c_str());
    return GK_OK;
}

// ---------------------------------------------------------- Rust formatting

// Rust's `{}` for f32: the shortest decimal that reads back as the same f32,
// written positionally (no exponent).  Used to reproduce the reference's
// "requantize scale ({s}) must be finite and > 0" message.
std::string rust_f32(float x) {
    if (std::isnan(x)) return "NaN";
    if (std::isinf(x)) return x > 0 ? "inf" : "-inf";
    if (x == 0.0f) return std::signbit(x) ? "-0" : "0";
    char buf[64];
    int prec = 1;
    for (; prec <= 9; ++prec) {
        snprintf(buf, sizeof buf, "%.*e", prec - 1, (double)x);
        if ((float)strtod(buf, nullptr) == x) break;
    }
    // buf = [-]d.ddde[+-]XX
    std::string s(buf);
    bool neg = s[0] == '-';
    if (neg) s = s.substr(1);
    size_t epos = s.find('e');
    int exp10 = atoi(s.c_str() + epos + 1);
    std::string digits;
    for (size_t i = 0; i < epos; ++i)
        if (s[i] != '.') digits += s[i];
    while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
    // value = 0.d1d2d3... * 10^(exp10+1)
    int point = exp10 + 1;
    std::string out;
    if (point <= 0) {
        out = "0." + std::string(-point, '0') + digits;
    } else if ((size_t)point >= digits.size()) {
        out = digits + std::string(point - digits.size(), '0');
    } else {
        out = digits.substr(0, point) + "." + digits.substr(point);
    }
    return neg ? "-" + out : out;
}

// ----------------------------------------------------------- view checks

// extent (src/api.rs:188-215): one past the highest element offset, or -1
// when a stride paired with a dimension > 1 is negative or arithmetic
// overflows.
bool extent(size_t rows, size_t cols, ptrdiff_t rs, ptrdiff_t cs, size_t *out) {
    if (rows == 0 || cols == 0) {
        *out = 0;
        return true;
    }
    __int128 lo = 0, hi = 0;
    const size_t dims[2] = {rows, cols};
    const ptrdiff_t strides[2] = {rs, cs};
    for (int t = 0; t < 2; ++t) {
        if (dims[t] > (size_t)PTRDIFF_MAX) return false;
        __int128 e = (__int128)(ptrdiff_t)(dims[t] - 1) * strides[t];
        if (e > PTRDIFF_MAX || e < PTRDIFF_MIN) return false;
        if (e < 0) lo += e; else hi += e;
        if (hi > PTRDIFF_MAX || lo < PTRDIFF_MIN) return false;
    }
    if (lo < 0) return false;
    if (hi + 1 > (__int128)SIZE_MAX) return false;
    *out = (size_t)hi + 1;
    return true;
}

// check_view (src/api.rs:197-213).
int check_view(size_t len, size_t rows, size_t cols, ptrdiff_t rs, ptrdiff_t cs,
               const char *name, const char *unchecked_name = "gemm_unchecked") {
    size_t need = 0;
    if (!extent(rows, cols, rs, cs, &need))
        return fail(GK_ERR_VIEW,
                    "gemmkit: %s view has negative strides or is too large to address; use %s",
                    name, unchecked_name);
    if (need > len)
        return fail(GK_ERR_VIEW,
                    "gemmkit: %s view of %zux%zu (strides %td,%td) needs %zu elements but slice "
                    "has %zu",
                    name, rows, cols, rs, cs, need, len);
    return GK_OK;
}

// self_aliases (src/api.rs:236-250).
bool self_aliases(size_t rows, size_t cols, ptrdiff_t rs, ptrdiff_t cs) {
    if (rows == 0 || cols == 0) return false;
    bool hr = rows > 1, hc = cols > 1;
    size_t ars = (size_t)(rs < 0 ? -(__int128)rs : rs), acs = (size_t)(cs < 0 ? -(__int128)cs : cs);
    if (!hr && !hc) return false;
    if (hr && !hc) return ars == 0;
    if (!hr && hc) return acs == 0;
    size_t sm_s, sm_d, big;
    if (ars <= acs) { sm_s = ars; sm_d = rows; big = acs; } else { sm_s = acs; sm_d = cols; big = ars; }
    __int128 span = (__int128)sm_s * sm_d;
    return sm_s == 0 || (__int128)big < span;
}

// overlaps_bytes (src/api.rs:520-536).
bool overlaps_bytes(const void *pa, size_t na, size_t sa, const void *pb, size_t nb, size_t sb) {
    uintptr_t a0 = (uintptr_t)pa, a1 = a0 + na * sa;
    uintptr_t b0 = (uintptr_t)pb, b1 = b0 + nb * sb;
    return a0 < b1 && b0 < a1;
}

// validate_gemm_views (src/api.rs:270-314).
int validate_gemm_views(const gk_mat_ref *a, const gk_mat_ref *b, const gk_mat_mut *c,
                        size_t si, size_t so) {
    if (!a || !b || !c) return fail(GK_ERR_ARG, "gemmkit: null view argument");
    if (a->cols != b->rows)
        return fail(GK_ERR_SHAPE, "gemmkit: A.cols (%zu) != B.rows (%zu)", a->cols, b->rows);
    if (a->rows != c->rows)
        return fail(GK_ERR_SHAPE, "gemmkit: A.rows (%zu) != C.rows (%zu)", a->rows, c->rows);
    if (b->cols != c->cols)
        return fail(GK_ERR_SHAPE, "gemmkit: B.cols (%zu) != C.cols (%zu)", b->cols, c->cols);
    int r;
    if ((r = check_view(a->len, a->rows, a->cols, a->rs, a->cs, "A"))) return r;
    if ((r = check_view(b->len, b->rows, b->cols, b->rs, b->cs, "B"))) return r;
    if ((r = check_view(c->len, c->rows, c->cols, c->rs, c->cs, "C"))) return r;
    if (self_aliases(c->rows, c->cols, c->rs, c->cs))
        return fail(GK_ERR_ALIAS,
                    "gemmkit: C view aliases itself (strides %td,%td map distinct elements to the "
                    "same memory); C must address each (i,j) uniquely",
                    c->rs, c->cs);
    if (overlaps_bytes(c->data, c->len, so, a->data, a->len, si) ||
        overlaps_bytes(c->data, c->len, so, b->data, b->len, si))
        return fail(GK_ERR_ALIAS, "gemmkit: C aliases A or B");
    return GK_OK;
}

// ------------------------------------------------------------ workspace

}  // namespace

struct gk_workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
    // Ordering of the arena across streams (the reference's &mut Workspace
    // has one user at a time, src/workspace.rs:53-60): the stream of the last
    // call that used it and an event recorded after that call's launches.
    hipStream_t last_stream = nullptr;
    hipEvent_t done = nullptr;
    bool recorded = false;
};

struct gk_packed_rhs {
    gk::InType in = gk::InType::I8;  // element type (PackedRhs<T>'s T)
    void *buf = nullptr;             // n x ld, k-contiguous rows (B transposed), zero padded
    size_t k = 0, n = 0;
    int64_t ld = 0;                  // row stride in elements
};

struct gk_packed_lhs {
    gk::InType in = gk::InType::F32;  // element type (PackedLhs<T>'s T)
    void *buf = nullptr;              // m x ld, k-contiguous rows of A, zero padded
    size_t m = 0, k = 0;
    int64_t ld = 0;                   // row stride in elements
};

namespace {

// The calling thread's default workspace (the reference's thread-local pool,
// src/workspace.rs:205-230): created on first use and released when a worker
// thread exits.  The main thread's arena is left to the process teardown,
// where the HIP runtime may already be gone.
// Waits until the arena's last user has finished with it (its event, not the
// whole device: other threads' queued work is not waited for).
void ws_quiesce(gk_workspace *ws) {
    if (ws->recorded) (void)hipEventSynchronize(ws->done);
    ws->recorded = false;
}

void ws_release(gk_workspace *ws) {
    if (tl_ws_recorded == &ws->recorded) tl_ws_recorded = nullptr;
    ws_quiesce(ws);
    if (ws->ptr) (void)hipFree(ws->ptr);
    ws->ptr = nullptr;
    ws->bytes = 0;
    if (ws->done) (void)hipEventDestroy(ws->done);
    ws->done = nullptr;
}

struct ThreadWs {
    gk_workspace *ws = nullptr;
    ~ThreadWs() {
        if (!ws) return;
        if ((pid_t)syscall(SYS_gettid) != getpid()) ws_release(ws);
        if (!ws->ptr) delete ws;
    }
};
thread_local ThreadWs tl_ws;

gk_workspace *resolve_ws(gk_workspace *ws) {
    if (ws) return ws;
    if (!tl_ws.ws) tl_ws.ws = new gk_workspace();
    return tl_ws.ws;
}

// True when the calling thread's launch stream is being captured into a HIP
// graph: nothing may allocate, free or synchronize then.
bool stream_capturing() {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(tl_stream, &st) != hipSuccess) return false;
    return st != hipStreamCaptureStatusNone;
}

// Returns a device region of at least `bytes`, growing the arena when needed.
// Growing synchronizes the device (work already queued may still read the old
// arena) and reallocates, which graph capture does not allow: under capture a
// call that needs more than the arena holds fails instead, and the caller
// reserves the arena beforehand (gk_workspace_with_capacity, or one eager call
// of the same shape).
int ws_reserve(gk_workspace *ws, size_t bytes, void **out) {
    const bool capturing = stream_capturing();
    if (ws->bytes < bytes) {
        if (stream_capturing())
            return fail(GK_ERR_NOMEM,
                        "gemmkit: the workspace must grow from %zu to %zu bytes during HIP graph "
                        "capture, which cannot allocate; size it before capturing "
                        "(gk_workspace_with_capacity, or one uncaptured call of the same shape)",
                        ws->bytes, bytes);
        size_t want = std::max(bytes, ws->bytes + ws->bytes / 2);
        want = (want + 0xFFFFF) & ~(size_t)0xFFFFF;
        if (ws->ptr) {
            // Work already queued may still read the old arena: wait for its
            // last user.
            if (ws->recorded) {
                hipError_t e = hipEventSynchronize(ws->done);
                if (e != hipSuccess) return hip_fail(e, "workspace grow");
                ws->recorded = false;
            }
            (void)hipFree(ws->ptr);
            ws->ptr = nullptr;
            ws->bytes = 0;
        }
        hipError_t e = hipMalloc(&ws->ptr, want);
        if (e != hipSuccess) {
            ws->ptr = nullptr;
            return fail(GK_ERR_NOMEM, "gemmkit: workspace allocation of %zu bytes failed", want);
        }
        ws->bytes = want;
    }
    // A call on another stream than the arena's last user first waits for
    // that user's work (its packs and partial sums live in the arena).
    // Captured calls follow the graph's own ordering: nothing is waited for
    // or recorded under capture.
    if (!capturing) {
        if (ws->recorded && ws->last_stream != tl_stream) {
            hipError_t e = hipStreamWaitEvent(tl_stream, ws->done, 0);
            if (e != hipSuccess) return hip_fail(e, "workspace stream order");
        }
        if (!ws->done) {
            hipError_t e = hipEventCreateWithFlags(&ws->done, hipEventDisableTiming);
            if (e != hipSuccess) return hip_fail(e, "workspace event");
        }
        ws->last_stream = tl_stream;
        tl_ws_event = ws->done;
        tl_ws_recorded = &ws->recorded;
    }
    *out = ws->ptr;
    return GK_OK;
}

int finish(const char *what) {
    hipError_t e = hipGetLastError();
    ws_mark_done();
    if (e != hipSuccess) return hip_fail(e, what);
    if (tl_sync) {
        e = hipStreamSynchronize(tl_stream);
        if (e != hipSuccess) return hip_fail(e, what);
    }
    return ok();
}

// ------------------------------------------------------------- dispatch

int64_t iabs64(int64_t v) { return v < 0 ? -v : v; }

// A kernel-frame operand: R rows, K contraction; element (r, p) at
// p_ + r*rs + p*ks (elements); batch element z adds z*bs.
struct Opnd {
    const void *p;
    int64_t rs, ks, bs;
};

// k-contiguous and 16-byte aligned, so the kernels can read it in place.  The
// kernels address a tile's rows as unsigned 32-bit offsets from its first row,
// so a negative row stride (legal on the unchecked tier) is never canonical:
// such an operand goes through the pack, which indexes in 64 bits.  A negative
// batch stride is fine (the kernels form each element's base in 64 bits).
bool canonical(const Opnd &o, int64_t R, int64_t K, size_t esz, int64_t batch) {
    if (K * (int64_t)esz % 16 != 0) return false;
    if (o.ks != 1 && K > 1) return false;
    if ((uintptr_t)o.p % 16 != 0) return false;
    if (R > 1 && o.rs < 0) return false;
    if (R > 1 && (o.rs * (int64_t)esz) % 16 != 0) return false;
    if (batch > 1 && (o.bs * (int64_t)esz) % 16 != 0) return false;
    return true;
}

int64_t round_up64(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Brings an operand into the k-contiguous layout, packing into `dst` when its
// own strides do not allow it.  Returns the (possibly new) operand.
int materialize(InType in, const Opnd &o, int64_t R, int64_t K, int64_t batch, uint8_t *dst,
                Opnd *out) {
    const size_t esz = in_size(in);
    const int64_t ld = round_up64(std::max<int64_t>(K, 1), 16 / (int64_t)esz);
    const int64_t nb = (batch > 1 && o.bs != 0) ? batch : 1;
    for (int64_t z = 0; z < nb; ++z) {
        const uint8_t *src = (const uint8_t *)o.p + z * o.bs * (int64_t)esz;
        hipError_t e = launch_pack(in, src, o.rs, o.ks, R, K, dst + z * R * ld * (int64_t)esz, ld,
                                   tl_stream);
        if (e != hipSuccess) return hip_fail(e, "pack");
    }
    *out = Opnd{dst, ld, 1, nb > 1 ? R * ld : 0};
    return GK_OK;
}

size_t pack_bytes(InType in, int64_t R, int64_t K, int64_t batch, const Opnd &o) {
    const size_t esz = in_size(in);
    const int64_t ld = round_up64(std::max<int64_t>(K, 1), 16 / (int64_t)esz);
    const int64_t nb = (batch > 1 && o.bs != 0) ? batch : 1;
    return (size_t)round_up64(nb * R * ld * (int64_t)esz, 256);
}

Tile env_tile(bool *forced) {
    const char *s = getenv("GEMMKIT_HIP_TILE");
    *forced = false;
    if (!s) return Tile::T256x256;
    *forced = true;
    if (!strcmp(s, "256x256")) return Tile::T256x256;
    if (!strcmp(s, "256x256w8")) return Tile::T256x256w8;
    if (!strcmp(s, "256x128o2")) return Tile::T256x128o2;
    if (!strcmp(s, "256x128")) return Tile::T256x128;
    if (!strcmp(s, "128x128")) return Tile::T128x128;
    if (!strcmp(s, "64x64")) return Tile::T64x64;
    if (!strcmp(s, "256x256k128")) return Tile::T256x256k128;
    if (!strcmp(s, "256x256w8k128")) return Tile::T256x256w8k128;
    if (!strcmp(s, "128x192k128")) return Tile::T128x192k128;
    if (!strcmp(s, "128x96k128o2")) return Tile::T128x96k128o2;
    if (!strcmp(s, "256x384w8k128")) return Tile::T256x384w8k128;
    if (!strcmp(s, "256x352w8k128")) return Tile::T256x352w8k128;
    if (!strcmp(s, "256x256w8m16")) return Tile::T256x256w8m16;
    if (!strcmp(s, "256x352w8m16")) return Tile::T256x352w8m16;
    *forced = false;
    return Tile::T256x256;
}

// GEMMKIT_HIP_SMALLF32=0 keeps small f32 products on split K.
bool small_f32_enabled() {
    const char *s = getenv("GEMMKIT_HIP_SMALLF32");
    return !(s && !strcmp(s, "0"));
}

// GEMMKIT_HIP_KSTREAM=0 keeps short contractions on the tile kernels.
bool kstream_enabled() {
    const char *s = getenv("GEMMKIT_HIP_KSTREAM");
    return !(s && !strcmp(s, "0"));
}

// GEMMKIT_HIP_SKINNY=0 keeps products with a short side of 2..8 on the
// wavefront-reduction GEMV instead of the matrix-core skinny kernel.
bool skinny_enabled() {
    const char *s = getenv("GEMMKIT_HIP_SKINNY");
    return !(s && !strcmp(s, "0"));
}

// Short sides where the wavefront GEMV streams faster than the matrix-core
// skinny kernel (graph-timed on 14336-row weights, five rotating copies):
// i8 with 2 vectors and 2..8 KiB rows (14336x4096: 11.1 against 12.7 us),
// f32 with 2..4 vectors and 4..8 KiB rows, where the skinny kernel spends
// four matrix-core operations per 16-byte chunk (14336x1024, 2 vectors:
// 11.0 against 18.4 us; 3 vectors: 14.0 against 17.8 us).  bf16 ties or
// loses.  Taken only when both operands are k-contiguous already, so the
// GEMV needs no pack launch.
static bool gemv_beats_skinny(InType in, int64_t short_side, int64_t kbytes) {
    if (in == InType::I8) return short_side == 2 && kbytes >= 2048 && kbytes <= 8192;
    if (in == InType::F32) return short_side <= 4 && kbytes >= 4096 && kbytes <= 8192;
    return false;
}

// Tile choice: the tile with the smallest makespan.  Tiles spread evenly over
// the CUs, so the busiest CU runs per_cu = ceil(tiles / CUs) of them, up to
// `occ` at a time.  A tile costs its main loop, BM*BN*kf / eff (kf: K bytes
// per row relative to 4096, times the f32 matrix cores' lower rate for f32
// inputs; eff[n-1] is the share of the CU's matrix-core peak n tiles sharing
// it deliver, times eff_i8 for int8 inputs, whose main loop draws more power
// per byte), plus its epilogue, BM*BN * c_epi(output kind) * epi (the tile's
// epilogue speed, epi_q8 for the requantizing one: eight waves per CU finish
// the arithmetic sooner), plus a fixed per-tile latency (first stages in
// flight).  A fraction `hide` of the epilogue and latency overlaps the next
// tile's main loop when a CU runs more than one; the last is never hidden.
// The constants are the fit of a tile sweep (profiles/tile_choice.md) to graph-timed
// runs of 17 shapes x 8 tiles (int8 i32 and requantized, bf16 with f32 and
// bf16 output, batched attention scores, f32; 1024^2 to 4096^3 and
// 2048 x 11008 x 4096): least squares on log time, then refined so the chosen
// tile is the best measured one on each shape.
struct TileCand { Tile t; int bm, bn, occ; double eff[2], eff_i8, hide, epi, epi_q8; };
static const TileCand kTileCands[] = {
    {Tile::T256x256, 256, 256, 1, {0.817513, 0.817513}, 1.0, 0.307445, 1.0, 1.0},
    {Tile::T256x256w8, 256, 256, 1, {0.798817, 0.798817}, 1.3, 0.1715, 1.144686, 0.968081},
    {Tile::T256x128o2, 256, 128, 2, {0.609198, 0.580406}, 0.950117, 0.464277, 0.66113, 0.740229},
    {Tile::T256x128, 256, 128, 1, {0.616949, 0.616949}, 1.026287, 0.0, 0.665666, 1.02864},
    {Tile::T128x128, 128, 128, 2, {0.616337, 0.540289}, 0.95272, 0.598733, 0.429867, 0.2},
    {Tile::T64x64, 64, 64, 2, {0.409374, 0.411763}, 0.709875, 0.812048, 0.2, 0.2},
    {Tile::T256x256k128, 256, 256, 1, {0.805722, 0.805722}, 1.3, 0.322672, 1.286801, 1.334919},
    {Tile::T256x256w8k128, 256, 256, 1, {0.821426, 0.821426}, 1.278928, 0.196392, 0.992329,
     0.969417},
    {Tile::T256x256w8m16, 256, 256, 1, {0.882658, 0.882658}, 1.3, 0.290227, 1.068566, 0.956933},
};

// The rest tile of a tail split run at a column pitch (T128x192k128): not a
// pick_tile candidate.  Its efficiencies are set between the 128x128 tile's
// and the 256-wide ones' (its operand reuse lies between theirs); they only
// rank it against the two 128-wide rests, and the layer shapes it is taken
// for were checked by measurement.
static const TileCand kPitchedRest = {Tile::T128x192k128, 128, 192, 1, {0.78, 0.78}, 1.0, 0.0,
                                      1.0, 0.6};
// The requantizing rest instead: 128 x 96 tiles, two per CU (each one's
// requantizing epilogue runs beside the other's main loop).  Measured on the
// 2048 x 11008 x 4096 layer: 103.2 against 106.8 us per call with the
// 128 x 192 rest; on i32 and bf16 output it loses (103.7 against 101.1 us,
// 161.4 against 155.2 us), so only requantized products take it.
static const TileCand kPitchedRestQ8 = {Tile::T128x96k128o2, 128, 96, 2, {0.78, 0.78}, 1.0, 0.0,
                                        1.0, 0.6};
// One round of 256 x 384 tiles at a column pitch (T256x384w8k128): when the
// 256-wide tiles need more than one round of the CUs and a pitch in
// (256, 384] covers the product in one, one launch of those tiles replaces
// the tail split.  Measured per-CU rate (the padded columns counted) equal to
// the 256 x 256 eight-wave tile's: 2048 x 11008 x 4096 i32 95.3 against
// 100.3 us, requantized 104.5 against 108.2 us, bf16 159.6 against 164.5 us,
// bf16 with f32 output 154.9 against 201.3 us, 4608 x 4608 x 4096 i32 91.8
// against 97.8 us.  f32 inputs lose (2048 x 11008 x 4096: 1379 against
// 1328 us) and never take it.
static const TileCand kRoundWide = {Tile::T256x384w8k128, 256, 384, 1, {0.821426, 0.821426},
                                    1.278928, 0.0, 0.992329, 0.969417};
// The same with 256 x 352 tiles (T256x352w8k128: the eight waves split the
// first 256 columns and a 96-column strip evenly), taken first for int8
// inputs where the pitch is at most 352: 2048 x 11008 x 4096 requantized
// 93.3 against 100.9 us with the 384-wide tile (103.6 with the tail split),
// i32 91.0 against 91.8 (97.0), 4608 x 4608 x 4096 86.9 against 88.6
// (95.2).  Its main loop reads 9 fragments per 11 MFMAs against the 384-wide
// tile's 7 per 12, and bf16 loses with it (161.6 against 155.8 us on the
// bf16 layer), so bf16 keeps the 384-wide tile.
static const TileCand kRoundStrip = {Tile::T256x352w8k128, 256, 352, 1, {0.821426, 0.821426},
                                     1.278928, 0.0, 0.992329, 0.969417};
// The 256 x 352 tile on 16x16 MFMAs (T256x352w8m16, mma16w.hip: 4 x 2 waves
// of 64 x 176, ping-pong schedule), taken before the 32x32 strip for int8
// inputs whenever the 16x16 tile is allowed (the same pitch rule).
static const TileCand kRoundStrip16 = {Tile::T256x352w8m16, 256, 352, 1, {0.882658, 0.882658},
                                       1.3, 0.0, 1.068566, 0.956933};

// Model cost of running an M x N (x batch) product with tile c, in the units
// of area / eff; `pitch` > 0: the tiles advance `pitch` columns at a time.
double tile_cost(const TileCand &c, int64_t M, int64_t N, int64_t batch, int64_t kbytes,
                 EpiKind kind, InType in, int64_t pitch = 0) {
    const double c_epi = kind == EpiKind::Q8 ? 0.602342
                         : kind == EpiKind::I32 ? 0.40104
                         : kind == EpiKind::F32 ? 0.251808 : 0.0;
    constexpr double kTileLatency = 11604.671;  // in the units of area / eff
    constexpr double kF32Rate = 4.530131;       // f32 main-loop cost per K byte vs i8/bf16
    const double kf = (double)std::max<int64_t>(kbytes, 64) / 4096.0 *
                      (in == InType::F32 ? kF32Rate : 1.0);
    const int64_t cus = g_num_cus > 0 ? g_num_cus : 256;
    const int64_t pn = pitch > 0 ? pitch : c.bn;
    const int64_t tiles = ((M + c.bm - 1) / c.bm) * ((N + pn - 1) / pn) * batch;
    const int64_t per_cu = (tiles + cus - 1) / cus;
    const int together = (int)std::min<int64_t>(per_cu, c.occ);
    const double area = (double)c.bm * c.bn;
    const double exposed = per_cu - c.hide * (per_cu - 1);
    const double eff = c.eff[together - 1] * (in == InType::I8 ? c.eff_i8 : 1.0);
    const double epi = kind == EpiKind::Q8 ? c.epi_q8 : c.epi;
    return per_cu * area * kf / eff + (area * c_epi * epi + kTileLatency) * exposed;
}

const TileCand &tile_cand(Tile t) {
    for (const TileCand &c : kTileCands)
        if (c.t == t) return c;
    if (t == kPitchedRest.t) return kPitchedRest;
    if (t == kPitchedRestQ8.t) return kPitchedRestQ8;
    if (t == kRoundWide.t) return kRoundWide;
    if (t == kRoundStrip.t) return kRoundStrip;
    if (t == kRoundStrip16.t) return kRoundStrip16;
    return kTileCands[0];
}

// The 16x16-MFMA tile (T256x256w8m16): int8 and bf16 inputs only (no f32
// variant).  Its bf16 sums take 32 k per instruction, the other tiles' 16,
// so bf16 results differ between it and them in the last bits: short bf16
// contractions stay on the 32x32 tiles, bit-identical to the streaming
// kernel that serves them.  GEMMKIT_HIP_M16=0 turns it off.
bool m16_allowed(InType in, int64_t kbytes) {
    const char *s = getenv("GEMMKIT_HIP_M16");
    if (s && !strcmp(s, "0")) return false;
    if (in == InType::F32) return false;
    return in == InType::I8 || kbytes > kstream_max_kbytes();
}

// m16: whether the 16x16-MFMA tile may be picked (on top of m16_allowed).
Tile pick_tile(int64_t M, int64_t N, int64_t batch, int64_t kbytes, EpiKind kind, InType in,
               double *cost_out = nullptr, bool m16 = true) {
    bool forced;
    Tile t = env_tile(&forced);
    if (forced) return t;
    double best = 1e300;
    Tile bt = Tile::T64x64;
    for (const TileCand &c : kTileCands) {
        if (c.t == Tile::T256x256w8m16 && (!m16 || !m16_allowed(in, kbytes))) continue;
        const double cost = tile_cost(c, M, N, batch, kbytes, kind, in);
        if (cost < best * 0.999) { best = cost; bt = c.t; }
    }
    if (cost_out) *cost_out = best;
    return bt;
}

// Tail split.  When a product's tiles take two or more rounds of the CUs and
// the last round is short, most CUs idle through it.  Cutting the kernel
// frame's N so that the first part fills the full rounds exactly and running
// the rest as a second launch with smaller tiles shortens that last round.
// The model decides: the split is taken when the two parts' modelled cost,
// plus one launch, beats the single launch.  Candidates for the rest: the
// 128-wide tiles (the model's efficiencies are fitted on full rounds; among
// those two it ranks the measured 2048 x 2816 x 4096 rests correctly), and
// 128 x 192 tiles at a column pitch that cuts the rest into exactly one round
// of the CUs (2048 x 2816: 16 x 16 tiles at a pitch of 176 columns).  Outputs
// do not change: every element's K order is the same in all tiles.
// GEMMKIT_HIP_TAILSPLIT=0 turns it off.
struct TailSplit { int64_t na; Tile ta, tb; int32_t pn_b; double cost; };

// Column pitch that runs an M x N rest as one round of tile c (occ tiles
// per CU): as many tile columns as the CUs leave per tile row, the pitch a
// multiple of 8 columns between half the tile's width and its width; 0 when
// there is none.
int32_t rest_pitch(const TileCand &c, int64_t M, int64_t N) {
    const int64_t cus = g_num_cus > 0 ? g_num_cus : 256;
    const int64_t tm = (M + c.bm - 1) / c.bm;
    const int64_t tn = cus * c.occ / tm;
    if (tn < 1) return 0;
    const int64_t p = ((N + tn - 1) / tn + 7) / 8 * 8;
    return (p >= c.bn / 2 && p <= c.bn) ? (int32_t)p : 0;
}
constexpr double kLaunchCost = 5000.0;  // one extra launch, in tile_cost units (~3 us)

bool tail_split_enabled() {
    const char *s = getenv("GEMMKIT_HIP_TAILSPLIT");
    return !(s && !strcmp(s, "0"));
}

// GEMMKIT_HIP_WIDE=0 turns off the one-round 256 x 384 plan.
bool wide_round_enabled() {
    const char *s = getenv("GEMMKIT_HIP_WIDE");
    return !(s && !strcmp(s, "0"));
}

bool plan_tail_split(int64_t M, int64_t N, int64_t kbytes, EpiKind kind, InType in, Tile t,
                     double cost_whole, TailSplit *out) {
    // bf16: the split's launches all sum in the 32x32 tiles' order, so the
    // split equals the one-round wide plan bit for bit.
    if (in == InType::BF16 && t == Tile::T256x256w8m16) t = Tile::T256x256w8k128;
    const TileCand &c = tile_cand(t);
    const int64_t cus = g_num_cus > 0 ? g_num_cus : 256;
    const int64_t tiles_m = (M + c.bm - 1) / c.bm, tiles_n = (N + c.bn - 1) / c.bn;
    const int64_t rounds = (tiles_m * tiles_n + cus - 1) / cus;
    if (rounds < 2) return false;
    const int64_t tn_a = (rounds - 1) * cus / tiles_m;  // tile columns of the full rounds
    if (tn_a <= 0 || tn_a >= tiles_n) return false;
    const int64_t na = tn_a * c.bn;
    const double cost_a = tile_cost(c, M, na, 1, kbytes, kind, in);
    double best_b = 1e300;
    Tile tb = Tile::T256x128;
    int32_t pn_b = 0;
    for (Tile cand : {Tile::T256x128, Tile::T128x128}) {
        const double cb = tile_cost(tile_cand(cand), M, N - na, 1, kbytes, kind, in);
        if (cb < best_b) { best_b = cb; tb = cand; }
    }
    const TileCand &pr = kind == EpiKind::Q8 ? kPitchedRestQ8 : kPitchedRest;
    if (const int32_t p = rest_pitch(pr, M, N - na)) {
        const double cb = tile_cost(pr, M, N - na, 1, kbytes, kind, in, p);
        if (cb < best_b) { best_b = cb; tb = pr.t; pn_b = p; }
    }
    if (cost_a + best_b + kLaunchCost >= cost_whole) return false;
    *out = TailSplit{na, t, tb, pn_b, cost_a + best_b + kLaunchCost};
    return true;
}

// The launch plan of an unsplit-K product: tile `ta` over kernel-frame
// columns [0, na) at column pitch pn_a (0: the tile's width), and, when
// na < N, tile `tb` over [na, N) at pitch pn_b.
struct MmaPlan { Tile ta; int32_t pn_a; int64_t na; Tile tb; int32_t pn_b; };

// ld_b: B^T's row stride in bytes.  The wide and strip tiles address 384 and
// 352 rows of B^T with 32-bit offsets from the panel's first row, so they are
// taken only when those rows plus the K bytes stay below 2^31 (the 256-row
// tiles are covered by the stride limit the caller enforces by packing).
bool wide_fits(const TileCand &c, int64_t ld_b, int64_t kbytes) {
    return panels_fit(1, c.bn, 0, ld_b, kbytes);
}

MmaPlan plan_mma(int64_t M, int64_t N, int64_t batch, int64_t kbytes, EpiKind kind, InType in,
                 int64_t ld_b = 0) {
    bool forced;
    env_tile(&forced);
    double cost = 0.0;
    // bf16 sums in the 16x16-MFMA tile's order differ in the last bits from
    // the 32x32 tiles' (all of which share one order), so a batch takes the
    // family its element's standalone plan takes: the 16x16 tile exactly
    // when that plan is the 16x16 tile, otherwise the best 32x32 tile for the
    // batch.  Every batched element then equals its standalone call bit for
    // bit (src/api/batched.rs:172-176).  int8 sums are exact in any order.
    bool m16 = true;
    if (in == InType::BF16 && batch > 1 && !forced) {
        const MmaPlan one = plan_mma(M, N, 1, kbytes, kind, in, ld_b);
        if (one.ta == Tile::T256x256w8m16) return MmaPlan{one.ta, 0, N, one.ta, 0};
        m16 = false;
    }
    const Tile t = pick_tile(M, N, batch, kbytes, kind, in, &cost, m16);
    if (forced) {
        int32_t p = 0;
        if (batch == 1 && (t == kRoundWide.t || t == kRoundStrip.t || t == kRoundStrip16.t))
            p = rest_pitch(tile_cand(t), M, N);
        // (a forced wide tile whose rows do not fit is refused at launch)
        return MmaPlan{t, p, N, t, 0};
    }
    MmaPlan plan{t, 0, N, t, 0};
    TailSplit ts;
    if (batch == 1 && tail_split_enabled() && plan_tail_split(M, N, kbytes, kind, in, t, cost, &ts)) {
        plan = MmaPlan{ts.ta, 0, ts.na, ts.tb, ts.pn_b};
        cost = ts.cost;
    }
    // One round of wide tiles: taken whenever it exists with at most 15% of
    // its columns padding (every such shape measured beat the tail split and
    // the single launch: the layers by 5-25%; the model, whose wide-tile
    // constants are the 256 x 256 eight-wave tile's, cannot rank them).
    if (batch == 1 && in != InType::F32 && wide_round_enabled()) {
        for (const TileCand *c : {&kRoundStrip16, &kRoundStrip, &kRoundWide}) {
            if (c == &kRoundStrip && in != InType::I8) continue;
            if (c == &kRoundStrip16 && (in != InType::I8 || !m16_allowed(in, kbytes))) continue;
            if (!wide_fits(*c, ld_b, kbytes)) continue;
            const int32_t p = rest_pitch(*c, M, N);
            if (p <= 256) continue;
            if (p * 100 >= c->bn * 85) {
                plan = MmaPlan{c->t, p, N, c->t, 0};
                break;
            }
        }
    }
    return plan;
}

// Split K: when the 64 x 64 tiles of one product leave most CUs idle and K is
// long, each tile's K is cut into ranges of at least kSplitMinBytes, enough
// of them for about two workgroups per CU.  The choice depends on the
// element shape only (never on the batch count), so a batched element equals
// the standalone product bit for bit.  GEMMKIT_HIP_SPLITK=0 turns it off.
constexpr int64_t kSplitMinBytes = 256;
constexpr int64_t kMaxSplits = 32;

int choose_splits(int64_t M, int64_t N, int64_t k, size_t esz) {
    const char *s = getenv("GEMMKIT_HIP_SPLITK");
    if (s && !strcmp(s, "0")) return 1;
    bool forced;
    (void)env_tile(&forced);
    if (forced) return 1;
    const int64_t kbytes = k * (int64_t)esz;
    const int64_t t64 = ((M + 63) / 64) * ((N + 63) / 64);
    const int64_t cus = g_num_cus > 0 ? g_num_cus : 256;
    if (2 * t64 > cus || kbytes < 2 * kSplitMinBytes) return 1;
    return (int)std::min<int64_t>(std::min<int64_t>(2 * cus / t64, kbytes / kSplitMinBytes),
                                  kMaxSplits);
}

// Device memory a call may use for packed operands and split-K partial sums:
// the workspace arena (grown on demand), or a fixed region handed down (the
// no-allocation entry point's static scratch, or the inner calls of a K-sliced
// product).
struct Region {
    gk_workspace *ws;      // used when fixed == nullptr
    uint8_t *fixed;
    size_t fixed_bytes;
};

int region_get(const Region &rg, size_t bytes, uint8_t **out) {
    if (rg.fixed) {
        if (bytes > rg.fixed_bytes)
            return fail(GK_ERR_NOMEM,
                        "gemmkit: this call needs %zu bytes of device scratch but its fixed "
                        "scratch holds %zu",
                        bytes, rg.fixed_bytes);
        *out = rg.fixed;
        return GK_OK;
    }
    void *p = nullptr;
    int r = ws_reserve(resolve_ws(rg.ws), bytes, &p);
    if (r) return r;
    *out = (uint8_t *)p;
    return GK_OK;
}

int64_t out_size(EpiKind kind) {
    return kind == EpiKind::Q8 ? 1 : (kind == EpiKind::BF16 ? 2 : 4);
}

const void *ptr_add(const void *p, int64_t bytes) {
    return p ? (const void *)((const uint8_t *)p + bytes) : p;
}

// Moves the per-channel vectors of `ep` (requantization scales and biases, or
// the fused bias) `off` channels on, when their axis is `axis`.
void channel_shift(EpiParams &ep, int32_t axis, int64_t off) {
    if (ep.axis != axis || off == 0) return;
    if (ep.scales) ep.scales += off;
    if (ep.bias) ep.bias += off;
    if (ep.fbias) ep.fbias = (const uint8_t *)ep.fbias + off * (ep.kind == EpiKind::BF16 ? 2 : 4);
}

// Rows or columns of the kernel frame one launch covers (tile indices and
// output coordinates are 32-bit in the kernels); longer sides run in pieces.
constexpr int64_t kMaxSide = int64_t(1) << 30;
// Partial-sum bytes of one split-K launch; a batch whose slabs need more runs
// in chunks of elements.
constexpr int64_t kSlabMax = int64_t(64) << 20;
// K bytes per piece of a K-sliced product (a multiple of every stage size).
constexpr int64_t kSliceBytes = int64_t(4) << 20;
// Longest K the wavefront GEMV takes in one launch.
constexpr int64_t kGemvMaxK = INT32_MAX;

int run_fit(const Region &rg, InType in, EpiParams ep, int64_t m, int64_t k, int64_t n,
            const void *a, int64_t rsa, int64_t csa, int64_t bsa, const void *b, int64_t rsb,
            int64_t csb, int64_t bsb, void *c, int64_t rsc, int64_t csc, int64_t bsc,
            int64_t batch, const gk_packed_rhs *packed, const gk_packed_lhs *packed_a);

// The shared core: C = epi(A*B) for every batch element.  `ep` comes in the
// user frame (rsc/csc of the user's C, axis 0 = per user row); m, k, n >= 1.
// Products larger than one launch takes are cut here, in the user frame, into
// pieces that each run as the standalone product would:
//   * more than kMaxGridZ batch elements: chunks of elements;
//   * more than kMaxSide rows or columns: bands of rows or columns (their
//     per-channel vectors move with them);
//   * a K too long for the kernels' 32-bit row offsets: K slices of
//     kSliceBytes whose products are summed in order into a native
//     accumulator slab (wrapping i32, or f32) -- the reference's own kc
//     slicing with beta = 1 after the first slice (src/driver.rs:725-730) --
//     and one pass then applies the call's epilogue to the sum.
int run_product(const Region &rg, InType in, EpiParams ep, int64_t m, int64_t k, int64_t n,
                const void *a, int64_t rsa, int64_t csa, int64_t bsa, const void *b,
                int64_t rsb, int64_t csb, int64_t bsb, void *c, int64_t rsc, int64_t csc,
                int64_t bsc, int64_t batch, const gk_packed_rhs *packed = nullptr,
                const gk_packed_lhs *packed_a = nullptr) {
    const int64_t esz = (int64_t)in_size(in), osz = out_size(ep.kind);
    int r;
    if (batch > kMaxGridZ) {
        for (int64_t z0 = 0; z0 < batch; z0 += kMaxGridZ) {
            const int64_t nb = std::min(kMaxGridZ, batch - z0);
            if ((r = run_product(rg, in, ep, m, k, n, ptr_add(a, z0 * bsa * esz), rsa, csa, bsa,
                                 ptr_add(b, z0 * bsb * esz), rsb, csb, bsb,
                                 (void *)ptr_add(c, z0 * bsc * osz), rsc, csc, bsc, nb, packed,
                                 packed_a)))
                return r;
        }
        return ok();
    }
    if (m > kMaxSide) {
        for (int64_t i0 = 0; i0 < m; i0 += kMaxSide) {
            const int64_t len = std::min(kMaxSide, m - i0);
            EpiParams e = ep;
            channel_shift(e, 0, i0);
            gk_packed_lhs pa;
            if (packed_a) {
                pa = *packed_a;
                pa.buf = (uint8_t *)pa.buf + i0 * pa.ld * esz;
                pa.m = (size_t)len;
            }
            if ((r = run_product(rg, in, e, len, k, n, ptr_add(a, i0 * rsa * esz), rsa, csa, bsa,
                                 b, rsb, csb, bsb, (void *)ptr_add(c, i0 * rsc * osz), rsc, csc,
                                 bsc, batch, packed, packed_a ? &pa : nullptr)))
                return r;
        }
        return ok();
    }
    if (n > kMaxSide) {
        for (int64_t j0 = 0; j0 < n; j0 += kMaxSide) {
            const int64_t len = std::min(kMaxSide, n - j0);
            EpiParams e = ep;
            channel_shift(e, 1, j0);
            gk_packed_rhs pb;
            if (packed) {
                pb = *packed;
                pb.buf = (uint8_t *)pb.buf + j0 * pb.ld * esz;
                pb.n = (size_t)len;
            }
            if ((r = run_product(rg, in, e, m, k, len, a, rsa, csa, bsa,
                                 ptr_add(b, j0 * csb * esz), rsb, csb, bsb,
                                 (void *)ptr_add(c, j0 * csc * osz), rsc, csc, bsc, batch,
                                 packed ? &pb : nullptr, packed_a)))
                return r;
        }
        return ok();
    }
    const bool gemv_route = std::min(m, n) <= 8;
    const bool too_long = gemv_route ? k > kGemvMaxK : k * esz > kMaxTileRowBytes;
    if (!too_long)
        return run_fit(rg, in, ep, m, k, n, a, rsa, csa, bsa, b, rsb, csb, bsb, c, rsc, csc, bsc,
                       batch, packed, packed_a);

    // K slices into a native slab (m x n row-major per element), then the
    // call's epilogue.  The slab and the slices' pack space are taken at once:
    // a slice's inner call packs both operands (their rows are longer than the
    // kernels address) into the space behind the slab.
    const int64_t S = kSliceBytes / esz;
    const size_t slab = (size_t)round_up64(batch * m * n * 4, 256);
    const size_t inner = (size_t)(round_up64(batch * m * S * esz, 256) +
                                  round_up64(batch * n * S * esz, 256) + kSlabMax);
    uint8_t *base = nullptr;
    if ((r = region_get(rg, slab + inner, &base))) return r;
    const Region in_rg{nullptr, base + slab, inner};
    EpiParams pe{};
    pe.kind = in == InType::I8 ? EpiKind::I32 : EpiKind::F32;
    pe.alpha_i = 1;
    pe.alpha_f = 1.0f;
    for (int64_t s0 = 0; s0 < k; s0 += S) {
        const int64_t len = std::min(S, k - s0);
        pe.beta_i = s0 ? 1 : 0;
        pe.beta_f = s0 ? 1.0f : 0.0f;
        gk_packed_rhs pb;
        gk_packed_lhs pa;
        if (packed) {
            pb = *packed;
            pb.buf = (uint8_t *)pb.buf + s0 * esz;
            pb.k = (size_t)len;
        }
        if (packed_a) {
            pa = *packed_a;
            pa.buf = (uint8_t *)pa.buf + s0 * esz;
            pa.k = (size_t)len;
        }
        if ((r = run_fit(in_rg, in, pe, m, len, n, ptr_add(a, s0 * csa * esz), rsa, csa, bsa,
                         ptr_add(b, s0 * rsb * esz), rsb, csb, bsb, base, n, 1, m * n, batch,
                         packed ? &pb : nullptr, packed_a ? &pa : nullptr)))
            return r;
    }
    EpiParams fe = ep;
    fe.c = c;
    fe.rsc = rsc;
    fe.csc = csc;
    fe.bsc = bsc;
    fe.vec4 = csc == 1 && (m == 1 || rsc % 4 == 0) && (batch <= 1 || bsc % 4 == 0) &&
              ((uintptr_t)c % (uintptr_t)(4 * osz)) == 0;
    hipError_t e = launch_split_reduce(in, base, 1, m, n, batch, fe, tl_stream);
    if (e != hipSuccess) return hip_fail(e, "k-slice epilogue launch");
    return finish("mfma gemm (K sliced)");
}

// One launch's worth of product (the limits above hold).
int run_fit(const Region &rg, InType in, EpiParams ep, int64_t m, int64_t k, int64_t n,
            const void *a, int64_t rsa, int64_t csa, int64_t bsa, const void *b, int64_t rsb,
            int64_t csb, int64_t bsb, void *c, int64_t rsc, int64_t csc, int64_t bsc,
            int64_t batch, const gk_packed_rhs *packed, const gk_packed_lhs *packed_a) {
    const size_t esz = in_size(in);
    // Orientation: the kernels write C row-major-ish (kernel column index the
    // fast one), so a column-major-ish C computes C^T = B^T A^T -- a swap of
    // roles only, both operands being read k-contiguous.
    const bool swap = iabs64(csc) > iabs64(rsc);
    Opnd A{a, rsa, csa, bsa};
    Opnd Bt{b, csb, rsb, bsb};  // B^T: n x k
    if (packed) Bt = Opnd{packed->buf, packed->ld, 1, 0};
    if (packed_a) A = Opnd{packed_a->buf, packed_a->ld, 1, 0};
    int64_t M = m, N = n;
    ep.c = c;
    ep.bsc = bsc;
    if (swap) {
        std::swap(A, Bt);
        std::swap(M, N);
        ep.rsc = csc;
        ep.csc = rsc;
        ep.axis ^= 1;
    } else {
        ep.rsc = rsc;
        ep.csc = csc;
    }

    // Route.  The matrix-core and skinny kernels address a tile's rows with
    // 32-bit offsets from its first row: 256 row strides plus a row must stay
    // below 2 GiB, so an operand with a longer row stride is packed (to rows
    // of K, which the caller keeps within that bound).
    const int64_t kbytes = k * (int64_t)esz;
    const bool a_ok = canonical(A, M, k, esz, batch) && A.rs * (int64_t)esz <= kMaxTileRowBytes;
    const bool b_ok = canonical(Bt, N, k, esz, batch) && Bt.rs * (int64_t)esz <= kMaxTileRowBytes;
    const bool k_fits = kbytes <= kMaxTileRowBytes;
    const int64_t short_side = std::min(M, N);
    // Skinny products: the short side's rows are the vectors.  One vector
    // streams best with the wavefront GEMV (a whole 1 KiB row segment per
    // load, no cross-wave exchange); 2..16 vectors go to the matrix-core
    // skinny kernel, which stages the vectors from any strides itself (only
    // the long operand must be k-contiguous), except the few short sides
    // gemv_beats_skinny names.  The choice depends on the shape and element
    // type only, so a batched element, a problem of a pointer-array batch and
    // the standalone call take the same kernel (and sum in the same order)
    // whatever their strides and alignment; the GEMV gets packed operands
    // when they are not k-contiguous.
    const bool vec_is_a = M <= N;
    const bool gemv_first = gemv_beats_skinny(in, short_side, kbytes);
    const bool skinny_ok = short_side >= 2 && short_side <= 16 && !gemv_first &&
                           skinny_enabled() && k_fits &&
                           skinny_lds_bytes(in, k, (int)short_side) <= kSkinnyLdsMax;
    const bool vector_route = skinny_ok || short_side <= 8;
    const bool pack_a = !a_ok && !(skinny_ok && vec_is_a);
    const bool pack_b = !b_ok && !(skinny_ok && !vec_is_a);
    // Split K.  Float products split by the element shape only (a batched
    // element sums in the same order as the standalone product); i8 sums do
    // not depend on the split (wrapping addition), so an i8 batch that fills
    // the CUs by itself is not split.
    int splits = vector_route ? 1 : choose_splits(M, N, k, esz);
    if (splits > 1 && in == InType::I8 && batch > 1 &&
        choose_splits(M, N * batch, k, esz) == 1)
        splits = 1;
    // K ranges of whole 64-byte stages; rounding up may leave fewer ranges,
    // every one of them non-empty.
    if (splits > 1) {
        const int64_t kc = round_up64((k + splits - 1) / splits, 64 / (int64_t)esz);
        splits = (int)((k + kc - 1) / kc);
    }
    // Small f32 products that split K (too few 64 x 64 tiles for the CUs)
    // run in one launch instead: a workgroup per 32 x 32 block with K split
    // over its 16 waves, operands read in place (no pack, no reduction
    // launch), when each wave's share stays short -- at most 256 k-pairs of
    // matrix-core work per round of blocks.  By the element shape only, so a
    // batched element takes the route of its standalone product.
    if (in == InType::F32 && splits > 1 && small_f32_enabled()) {
        const int64_t cus = g_num_cus > 0 ? g_num_cus : 256;
        const int64_t blocks = ((M + 31) / 32) * ((N + 31) / 32);
        if ((blocks + cus - 1) / cus * ((k + 31) / 32) <= 256) {
            const SmallArgs sa{A.p, Bt.p, A.rs, A.ks, Bt.rs, Bt.ks, A.bs, Bt.bs,
                               (int32_t)M, (int32_t)N, (int32_t)k, (int32_t)batch};
            hipError_t e = launch_small_f32(sa, ep, tl_stream);
            if (e != hipSuccess) return hip_fail(e, "small f32 gemm launch");
            return finish("small f32 gemm");
        }
    }
    const size_t a_bytes = pack_a ? pack_bytes(in, M, k, batch, A) : 0;
    const size_t b_bytes = pack_b ? pack_bytes(in, N, k, batch, Bt) : 0;
    // In a fixed scratch region an i8 product takes fewer K ranges when the
    // partial sums would not fit beside the packed operands (its bits do not
    // depend on the split).
    if (rg.fixed && in == InType::I8 && splits > 1) {
        const int64_t avail = (int64_t)rg.fixed_bytes - (int64_t)(a_bytes + b_bytes);
        const int64_t fit = avail > 0 ? (avail & ~(int64_t)255) / (M * N * 4) : 0;
        if (fit < splits) {
            splits = fit >= 2 ? (int)fit : 1;
            const int64_t kc = round_up64((k + splits - 1) / splits, 64 / (int64_t)esz);
            splits = (int)((k + kc - 1) / kc);
        }
    }
    const int64_t kchunk = splits > 1 ? round_up64((k + splits - 1) / splits, 64 / (int64_t)esz) : k;
    // Batch elements per split-K launch: as many as kSlabMax of partial sums
    // holds (at least one).
    const int64_t elem_part = (int64_t)splits * M * N * 4;
    const int64_t zchunk = splits > 1 ? std::max<int64_t>(1, std::min(batch, kSlabMax / elem_part)) : batch;
    const size_t part_bytes = splits > 1 ? (size_t)round_up64(zchunk * elem_part, 256) : 0;

    uint8_t *part = nullptr;
    if (pack_a || pack_b || part_bytes) {
        uint8_t *dst = nullptr;
        int r = region_get(rg, a_bytes + b_bytes + part_bytes, &dst);
        if (r) return r;
        if (pack_a && (r = materialize(in, A, M, k, batch, dst, &A))) return r;
        if (pack_b && (r = materialize(in, Bt, N, k, batch, dst + a_bytes, &Bt))) return r;
        part = dst + a_bytes + b_bytes;
    }

    hipError_t e;
    if (vector_route) {
        // Skinny route: the short side's rows are the vectors, streamed
        // against the long side's rows (matrix-core kernel up to 16 vectors
        // when the vectors fit in LDS, else the wavefront-reduction GEMV),
        // every batch element in one launch (grid y).
        GemvArgs g{};
        EpiParams eg = ep;
        const Opnd &mat = vec_is_a ? Bt : A;
        const Opnd &vec = vec_is_a ? A : Bt;
        if (vec_is_a) {
            g.R = (int32_t)N; g.nvec = (int32_t)M;
        } else {
            g.R = (int32_t)M; g.nvec = (int32_t)N;
            std::swap(eg.rsc, eg.csc);
            eg.axis ^= 1;
        }
        g.mat = mat.p; g.ld = mat.rs; g.bsm = mat.bs;
        g.vec = vec.p; g.vld = vec.rs; g.vks = vec.ks; g.bsv = vec.bs;
        g.K = (int32_t)k;
        g.cus = g_num_cus;
        g.batch = (int32_t)batch;
        e = skinny_ok ? launch_skinny(in, g, eg, tl_stream) : launch_gemv(in, g, eg, tl_stream);
        if (e != hipSuccess) return hip_fail(e, skinny_ok ? "skinny launch" : "gemv launch");
        return finish(skinny_ok ? "skinny" : "gemv");
    }

    // Whole 4-element output chunks can go out as one vector access when C is
    // unit-stride along the kernel's columns and every chunk start is aligned.
    const int64_t osz = out_size(ep.kind);
    ep.vec4 = ep.csc == 1 && (M == 1 || ep.rsc % 4 == 0) && (batch <= 1 || bsc % 4 == 0) &&
              ((uintptr_t)c % (uintptr_t)(4 * osz)) == 0;
    MmaArgs args{};
    args.a = A.p;
    args.b = Bt.p;
    args.lda = A.rs;
    args.ldb = Bt.rs;
    args.bsa = A.bs;
    args.bsb = Bt.bs;
    args.M = (int32_t)M;
    args.N = (int32_t)N;
    args.K = (int32_t)k;
    args.batch = (int32_t)batch;
    args.splits = 1;
    if (splits > 1) {
        // Partial sums of each K range into their own slab (i32 for i8
        // inputs, f32 otherwise), then one pass sums the slabs in range order
        // and applies the call's epilogue; zchunk batch elements at a time.
        args.splits = splits;
        args.kchunk = (int32_t)kchunk;
        EpiParams pe{};
        pe.kind = in == InType::I8 ? EpiKind::I32 : EpiKind::F32;
        pe.alpha_i = 1;
        pe.alpha_f = 1.0f;
        pe.c = part;
        pe.rsc = N;
        pe.csc = 1;
        pe.bsc = M * N;
        pe.vec4 = N % 4 == 0;
        for (int64_t z0 = 0; z0 < batch; z0 += zchunk) {
            MmaArgs az = args;
            az.batch = (int32_t)std::min(zchunk, batch - z0);
            az.a = ptr_add(A.p, z0 * A.bs * (int64_t)esz);
            az.b = ptr_add(Bt.p, z0 * Bt.bs * (int64_t)esz);
            EpiParams ez = ep;
            ez.c = (void *)ptr_add(ep.c, z0 * bsc * osz);
            e = launch_mma(in, Tile::T64x64, az, pe, tl_stream);
            if (e != hipSuccess) return hip_fail(e, "mfma launch");
            e = launch_split_reduce(in, part, splits, M, N, az.batch, ez, tl_stream);
            if (e != hipSuccess) return hip_fail(e, "split reduce launch");
        }
        return finish("mfma gemm (split K)");
    }
    bool forced;
    env_tile(&forced);
    // Short contractions are bound by the output write: the streaming kernel
    // overlaps each tile's write with the next tile's loads (same results as
    // the tile kernels, bit for bit).
    if (!forced && kstream_enabled() && ep.kind != EpiKind::Q8 && kbytes <= kstream_max_kbytes() &&
        M >= 128 && N >= 128) {
        e = launch_kstream(in, args, ep, g_num_cus, tl_stream);
        if (e != hipSuccess) return hip_fail(e, "kstream launch");
        return finish("mfma gemm (short K)");
    }
    const MmaPlan plan = plan_mma(M, N, batch, kbytes, ep.kind, in, Bt.rs * (int64_t)esz);
    if (plan.na < N) {
        // Tail split: kernel-frame columns [0, na) with the first tile,
        // [na, N) with the rest's (at its column pitch, if any): B^T rows, C
        // columns and, for per-column channels, the scales, biases and fused
        // biases start na further on.
        MmaArgs a1 = args, a2 = args;
        a1.N = (int32_t)plan.na;
        a1.pn = plan.pn_a;
        a2.N = (int32_t)(N - plan.na);
        a2.pn = plan.pn_b;
        a2.b = (const uint8_t *)Bt.p + plan.na * Bt.rs * (int64_t)esz;
        EpiParams e2 = ep;
        e2.c = (uint8_t *)ep.c + plan.na * ep.csc * osz;
        channel_shift(e2, 1, plan.na);
        e = launch_mma(in, plan.ta, a1, ep, tl_stream);
        if (e != hipSuccess) return hip_fail(e, "mfma launch");
        e = launch_mma(in, plan.tb, a2, e2, tl_stream);
        if (e != hipSuccess) return hip_fail(e, "mfma launch");
        return finish("mfma gemm (tail split)");
    }
    MmaArgs aw = args;
    aw.pn = plan.pn_a;
    e = launch_mma(in, plan.ta, aw, ep, tl_stream);
    if (e != hipSuccess) return hip_fail(e, "mfma launch");
    return finish("mfma gemm");
}

// Sizes the reference accepts (it fails closed only where its pack sizes
// overflow, src/workspace.rs:25-45): every dimension and element count must be
// addressable with signed 64-bit element offsets.
bool dims_fit(size_t m, size_t k, size_t n, size_t batch) {
    const size_t lim = (size_t)INT64_MAX / 16;
    return m <= lim && k <= lim && n <= lim && batch <= lim;
}

// Calls fn(z0, nb, i0, mm, j0, nn) over blocks of a (batch x) m x n user-frame
// C of at most kMaxGridZ elements, kMaxSide rows and kMaxSide columns (the
// element-wise fill kernels index one block per launch).
template <typename F>
hipError_t for_c_blocks(int64_t m, int64_t n, int64_t batch, F fn) {
    for (int64_t z0 = 0; z0 < batch; z0 += kMaxGridZ)
        for (int64_t i0 = 0; i0 < m; i0 += kMaxSide)
            for (int64_t j0 = 0; j0 < n; j0 += kMaxSide) {
                hipError_t e = fn(z0, std::min(kMaxGridZ, batch - z0), i0,
                                  std::min(kMaxSide, m - i0), j0, std::min(kMaxSide, n - j0));
                if (e != hipSuccess) return e;
            }
    return hipSuccess;
}

// Degenerate C <- beta*C (k == 0 or alpha == 0).
int scale_c(EpiKind kind, void *c, size_t m, size_t n, ptrdiff_t rsc, ptrdiff_t csc,
            size_t batch, ptrdiff_t bsc, int32_t beta_i, float beta_f) {
    bool one = (kind == EpiKind::I32) ? beta_i == 1 : beta_f == 1.0f;
    if (one) return ok();
    const int64_t osz = out_size(kind);
    hipError_t e = for_c_blocks((int64_t)m, (int64_t)n, (int64_t)batch,
                                [&](int64_t z0, int64_t nb, int64_t i0, int64_t mm, int64_t j0,
                                    int64_t nn) {
        void *cb = (void *)ptr_add(c, (z0 * bsc + i0 * rsc + j0 * csc) * osz);
        return launch_scale_c(kind, cb, mm, nn, rsc, csc, nb, bsc, beta_i, beta_f, tl_stream);
    });
    if (e != hipSuccess) return hip_fail(e, "scale_c launch");
    return finish("scale_c");
}

// The fused degenerate map over a (batch x) m x n user-frame C (`ep` in the
// user frame).
hipError_t fused_fill_blocks(const EpiParams &ep, int64_t m, int64_t n, int64_t batch) {
    const int64_t osz = out_size(ep.kind);
    return for_c_blocks(m, n, batch, [&](int64_t z0, int64_t nb, int64_t i0, int64_t mm,
                                         int64_t j0, int64_t nn) {
        EpiParams e = ep;
        e.c = (void *)ptr_add(ep.c, (z0 * ep.bsc + i0 * ep.rsc + j0 * ep.csc) * osz);
        channel_shift(e, 0, i0);
        channel_shift(e, 1, j0);
        return launch_fused_fill(e, mm, nn, nb, tl_stream);
    });
}

// The k == 0 requant fill over an m x n user-frame C.
hipError_t requant_fill_blocks(const EpiParams &ep, int64_t m, int64_t n) {
    return for_c_blocks(m, n, 1, [&](int64_t, int64_t, int64_t i0, int64_t mm, int64_t j0,
                                     int64_t nn) {
        EpiParams e = ep;
        e.c = (void *)ptr_add(ep.c, i0 * ep.rsc + j0 * ep.csc);
        channel_shift(e, 0, i0);
        channel_shift(e, 1, j0);
        return launch_requant_fill(e, mm, nn, tl_stream);
    });
}

EpiParams epi_int(int32_t alpha, int32_t beta) {
    EpiParams ep{};
    ep.kind = EpiKind::I32;
    ep.alpha_i = alpha;
    ep.beta_i = beta;
    return ep;
}

EpiParams epi_float(EpiKind kind, float alpha, float beta) {
    EpiParams ep{};
    ep.kind = kind;
    ep.alpha_f = alpha;
    ep.beta_f = beta;
    return ep;
}

float bf16_to_f32(gk_bf16 h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// ---- i8 -> i32 core (execute_int, src/dispatch/int.rs:131-148)
int exec_i8(gk_workspace *ws, size_t m, size_t k, size_t n, int32_t alpha, const int8_t *a,
            ptrdiff_t rsa, ptrdiff_t csa, const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
            int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc,
            const gk_packed_rhs *packed = nullptr, const Region *fixed = nullptr) {
    int r;
    if ((r = device_init())) return r;
    if (m == 0 || n == 0) return ok();
    if (!dims_fit(m, k, n, 1)) return fail(GK_ERR_OVERFLOW, "gemmkit: GEMM is too large; the pack workspace size overflows usize");
    if (k == 0 || alpha == 0) return scale_c(EpiKind::I32, c, m, n, rsc, csc, 1, 0, beta, 0.f);
    return run_product(fixed ? *fixed : Region{ws, nullptr, 0}, InType::I8, epi_int(alpha, beta),
                       m, k, n, a, rsa, csa, 0, b, rsb, csb,
                       0, c, rsc, csc, 0, 1, packed);
}

// A lowered fused epilogue (to_fused_epi_raw, src/api.rs:354-380): the bias
// pointer (f32, or bf16 for bf16 output) with its user-frame axis, and the
// activation.
struct FusedSpec {
    const void *bias;
    int32_t dim;    // GK_BIAS_PER_ROW / GK_BIAS_PER_COL
    int32_t act;    // GK_ACT_NONE / GK_ACT_RELU / GK_ACT_LEAKY_RELU
    float slope;
};

// The raw tier's enum arguments: values outside the reference's enums.
int check_fused_enums(const FusedSpec &fx) {
    if (fx.bias && fx.dim != GK_BIAS_PER_ROW && fx.dim != GK_BIAS_PER_COL)
        return fail(GK_ERR_ARG, "gemmkit: bias dim (%d) must be 0 (PerRow) or 1 (PerCol)", fx.dim);
    if (fx.act != GK_ACT_NONE && fx.act != GK_ACT_RELU && fx.act != GK_ACT_LEAKY_RELU)
        return fail(GK_ERR_ARG,
                    "gemmkit: activation (%d) must be 0 (none), 1 (Relu) or 2 (LeakyRelu)", fx.act);
    return GK_OK;
}

// ---- float-family core (execute, src/dispatch.rs:345-358; execute_fused,
// src/dispatch/float.rs:661-680; execute_packed(_fused), src/dispatch.rs:366-380,
// src/dispatch/float.rs:692-735)
int exec_float(gk_workspace *ws, InType in, EpiKind kind, size_t batch, size_t m, size_t k,
               size_t n, float alpha, const void *a, ptrdiff_t rsa, ptrdiff_t csa, ptrdiff_t bsa,
               const void *b, ptrdiff_t rsb, ptrdiff_t csb, ptrdiff_t bsb, float beta, void *c,
               ptrdiff_t rsc, ptrdiff_t csc, ptrdiff_t bsc, const FusedSpec *fx = nullptr,
               const gk_packed_rhs *packed = nullptr, const gk_packed_lhs *packed_a = nullptr) {
    int r;
    if ((r = device_init())) return r;
    if (fx && (r = check_fused_enums(*fx))) return r;
    if (batch == 0 || m == 0 || n == 0) return ok();
    if (!dims_fit(m, k, n, batch)) return fail(GK_ERR_OVERFLOW, "gemmkit: GEMM is too large; the pack workspace size overflows usize");
    EpiParams ep = epi_float(kind, alpha, beta);
    if (fx) {
        ep.fbias = fx->bias;
        ep.axis = fx->bias ? fx->dim : 0;
        ep.act = fx->act;
        ep.slope = fx->slope;
        ep.fused = (fx->bias != nullptr || fx->act != GK_ACT_NONE) ? 1 : 0;
    }
    if (k == 0 || alpha == 0.0f) {
        if (!ep.fused) return scale_c(kind, c, m, n, rsc, csc, batch, bsc, 0, beta);
        ep.c = c;
        ep.rsc = rsc;
        ep.csc = csc;
        ep.bsc = bsc;
        hipError_t e = fused_fill_blocks(ep, (int64_t)m, (int64_t)n, (int64_t)batch);
        if (e != hipSuccess) return hip_fail(e, "fused fill launch");
        return finish("fused fill");
    }
    return run_product(Region{ws, nullptr, 0}, in, ep, m, k, n, a, rsa, csa, bsa, b, rsb, csb, bsb,
                       c, rsc, csc, bsc,
                       batch, packed, packed_a);
}

// ---- requant core (execute_int_requant, src/dispatch/int.rs:672-700)
int exec_requant(gk_workspace *ws, size_t m, size_t k, size_t n, const int8_t *a, ptrdiff_t rsa,
                 ptrdiff_t csa, const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb, float scale,
                 const float *scales, int32_t zp, const int32_t *bias, int32_t axis, int32_t act,
                 int32_t lo, int32_t hi, void *c, ptrdiff_t rsc, ptrdiff_t csc,
                 const gk_packed_rhs *packed = nullptr) {
    int r;
    if ((r = device_init())) return r;
    if (axis != GK_AXIS_ROW && axis != GK_AXIS_COL)
        return fail(GK_ERR_ARG, "gemmkit: requantize axis (%d) must be 0 (per-row) or 1 (per-col)", axis);
    if (act != GK_ACT_NONE && act != GK_ACT_RELU)
        return fail(GK_ERR_ARG, "gemmkit: requantize act (%d) must be 0 (none) or 1 (relu)", act);
    if (m == 0 || n == 0) return ok();
    if (!dims_fit(m, k, n, 1)) return fail(GK_ERR_OVERFLOW, "gemmkit: GEMM is too large; the pack workspace size overflows usize");
    EpiParams ep{};
    ep.kind = EpiKind::Q8;
    ep.scale = scale;
    ep.scales = scales;
    ep.bias = bias;
    ep.axis = axis;
    ep.zp = zp;
    ep.lo = (act == GK_ACT_RELU) ? std::max(lo, zp) : lo;
    ep.hi = hi;
    if (k == 0) {
        ep.c = c;
        ep.rsc = rsc;
        ep.csc = csc;
        hipError_t e = requant_fill_blocks(ep, (int64_t)m, (int64_t)n);
        if (e != hipSuccess) return hip_fail(e, "requant fill launch");
        return finish("requant fill");
    }
    return run_product(Region{ws, nullptr, 0}, InType::I8, ep, m, k, n, a, rsa, csa, 0, b, rsb,
                       csb, 0, c, rsc, csc,
                       0, 1, packed);
}

// Per-channel scale vectors this thread has checked outside graph capture
// (the last few, by device pointer and length).
thread_local std::vector<std::pair<const float *, size_t>> tl_checked_scales;

bool scales_checked(const float *p, size_t len) {
    for (const auto &e : tl_checked_scales)
        if (e.first == p && e.second == len) return true;
    return false;
}

void note_scales_checked(const float *p, size_t len) {
    if (scales_checked(p, len)) return;
    if (tl_checked_scales.size() >= 64) tl_checked_scales.erase(tl_checked_scales.begin());
    tl_checked_scales.emplace_back(p, len);
}

// requant_scale / requant_bias / zero-point checks (src/adapter.rs:190-273,
// src/api/int8.rs:291-295, :506-510).  `chan` is the channel count of the
// chosen axis; `axis_name` is "A.rows" for the reference's per-row vectors.
int validate_requant(const gk_requantize *req, const gk_mat_mut *c, size_t m, size_t n, bool u8) {
    if (!req) return fail(GK_ERR_ARG, "gemmkit: null requantize argument");
    if (req->axis != GK_AXIS_ROW && req->axis != GK_AXIS_COL)
        return fail(GK_ERR_ARG, "gemmkit: requantize axis (%d) must be 0 (per-row) or 1 (per-col)",
                    req->axis);
    if (req->act != GK_ACT_NONE && req->act != GK_ACT_RELU)
        return fail(GK_ERR_ARG, "gemmkit: requantize act (%d) must be 0 (none) or 1 (relu)", req->act);
    const size_t chan = req->axis == GK_AXIS_ROW ? m : n;
    const char *axis_name = req->axis == GK_AXIS_ROW ? "A.rows" : "B.cols";
    if (!req->scales) {
        float s = req->scale;
        if (!(std::isfinite(s) && s > 0.0f))
            return fail(GK_ERR_ARG, "gemmkit: requantize scale (%s) must be finite and > 0",
                        rust_f32(s).c_str());
    } else {
        if (req->scales_len != chan)
            return fail(GK_ERR_SHAPE, "gemmkit: requantize scales length (%zu) != %s (%zu)",
                        req->scales_len, axis_name, chan);
        if (overlaps_bytes(c->data, c->len, 1, req->scales, req->scales_len, 4))
            return fail(GK_ERR_ALIAS, "gemmkit: requantize scales overlap C");
        // The scale values live in device memory: copy them back to check
        // (the reference checks them when its RequantScale is built, and the
        // slice stays borrowed, so they cannot change afterwards).  Under HIP
        // graph capture nothing can be copied back: a capture accepts the
        // scales an uncaptured call on this thread has already checked (same
        // pointer and length), and fails with a clear error otherwise.
        if (chan > 0 && stream_capturing()) {
            if (!scales_checked(req->scales, chan))
                return fail(GK_ERR_ARG,
                            "gemmkit: requantize scales cannot be checked during HIP graph "
                            "capture; make one uncaptured call with the same scales first, or use "
                            "the _unchecked entry");
        } else if (chan > 0) {
            float *h = (float *)malloc(chan * sizeof(float));
            if (!h) return fail(GK_ERR_NOMEM, "gemmkit: host allocation failed");
            hipError_t e = hipMemcpy(h, req->scales, chan * sizeof(float), hipMemcpyDeviceToHost);
            if (e != hipSuccess) {
                free(h);
                return hip_fail(e, "requantize scale check");
            }
            for (size_t i = 0; i < chan; ++i) {
                if (!(std::isfinite(h[i]) && h[i] > 0.0f)) {
                    std::string t = rust_f32(h[i]);
                    free(h);
                    return fail(GK_ERR_ARG, "gemmkit: requantize scale (%s) must be finite and > 0",
                                t.c_str());
                }
            }
            free(h);
            note_scales_checked(req->scales, chan);
        }
    }
    if (u8) {
        if (req->zero_point < 0 || req->zero_point > 255)
            return fail(GK_ERR_ARG, "gemmkit: requantize zero_point (%d) out of u8 range [0, 255]",
                        req->zero_point);
    } else if (req->zero_point < -128 || req->zero_point > 127) {
        return fail(GK_ERR_ARG, "gemmkit: requantize zero_point (%d) out of i8 range [-128, 127]",
                    req->zero_point);
    }
    if (req->bias) {
        if (req->bias_len != chan)
            return fail(GK_ERR_SHAPE, "gemmkit: requantize bias length (%zu) != %s (%zu)",
                        req->bias_len, axis_name, chan);
        if (overlaps_bytes(c->data, c->len, 1, req->bias, req->bias_len, 4))
            return fail(GK_ERR_ALIAS, "gemmkit: requantize bias overlaps C");
    }
    return GK_OK;
}

int requant_checked(gk_workspace *ws, const gk_mat_ref *a, const gk_mat_ref *b,
                    const gk_packed_rhs *packed, const gk_requantize *req, const gk_mat_mut *c,
                    bool u8) {
    int r;
    if (packed) {
        if (!a || !c) return fail(GK_ERR_ARG, "gemmkit: null view argument");
        if (a->cols != packed->k)
            return fail(GK_ERR_SHAPE, "gemmkit: A.cols (%zu) != packed B.rows (%zu)", a->cols, packed->k);
        if (packed->n != c->cols)
            return fail(GK_ERR_SHAPE, "gemmkit: packed B.cols (%zu) != C.cols (%zu)", packed->n, c->cols);
        if (a->rows != c->rows)
            return fail(GK_ERR_SHAPE, "gemmkit: A.rows (%zu) != C.rows (%zu)", a->rows, c->rows);
        if ((r = check_view(a->len, a->rows, a->cols, a->rs, a->cs, "A"))) return r;
        if ((r = check_view(c->len, c->rows, c->cols, c->rs, c->cs, "C"))) return r;
        if (self_aliases(c->rows, c->cols, c->rs, c->cs))
            return fail(GK_ERR_ALIAS,
                        "gemmkit: C view aliases itself (strides %td,%td map distinct elements to "
                        "the same memory); C must address each (i,j) uniquely",
                        c->rs, c->cs);
        if (overlaps_bytes(c->data, c->len, 1, a->data, a->len, 1))
            return fail(GK_ERR_ALIAS, "gemmkit: C aliases A");
    } else if ((r = validate_gemm_views(a, b, c, 1, 1))) {
        return r;
    }
    const size_t m = a->rows, k = a->cols, n = c->cols;
    if ((r = validate_requant(req, c, m, n, u8))) return r;
    const int8_t *bp = packed ? nullptr : (const int8_t *)b->data;
    return exec_requant(ws, m, k, n, (const int8_t *)a->data, a->rs, a->cs, bp,
                        packed ? 0 : b->rs, packed ? 0 : b->cs, req->scale, req->scales,
                        req->zero_point, req->bias, req->axis, req->act, u8 ? 0 : -128,
                        u8 ? 255 : 127, c->data, c->rs, c->cs, packed);
}

// check_batched_view (src/api/batched.rs:31-69); returns the element extent.
int check_batched_view(size_t len, size_t rows, size_t cols, ptrdiff_t rs, ptrdiff_t cs,
                       size_t batch, ptrdiff_t bs, const char *name, size_t *ext) {
    size_t e = 0;
    if (!extent(rows, cols, rs, cs, &e))
        return fail(GK_ERR_VIEW,
                    "gemmkit: %s view has negative strides or is too large to address; use the "
                    "unchecked API",
                    name);
    size_t last_base = 0;
    if (batch > 1) {
        if (bs < 0)
            return fail(GK_ERR_VIEW, "gemmkit: %s batch stride (%td) must be non-negative", name, bs);
        __int128 lb = (__int128)(batch - 1) * (size_t)bs;
        last_base = lb > (__int128)SIZE_MAX ? SIZE_MAX : (size_t)lb;
    }
    size_t need = last_base > SIZE_MAX - e ? SIZE_MAX : last_base + e;
    if (need > len)
        return fail(GK_ERR_VIEW,
                    "gemmkit: %s batched view (%zu\xC3\x97 %zux%zu, batch stride %td) needs %zu "
                    "elements but slice has %zu",
                    name, batch, rows, cols, bs, need, len);
    *ext = e;
    return GK_OK;
}

// validate_batched_views (src/api/batched.rs:78-163).
int validate_batched_views(size_t batch, const gk_mat_ref *a, ptrdiff_t a_bs, const gk_mat_ref *b,
                           ptrdiff_t b_bs, const gk_mat_mut *c, ptrdiff_t c_bs, size_t si,
                           size_t so) {
    if (!a || !b || !c) return fail(GK_ERR_ARG, "gemmkit: null view argument");
    if (a->cols != b->rows)
        return fail(GK_ERR_SHAPE, "gemmkit: A.cols (%zu) != B.rows (%zu)", a->cols, b->rows);
    if (a->rows != c->rows)
        return fail(GK_ERR_SHAPE, "gemmkit: A.rows (%zu) != C.rows (%zu)", a->rows, c->rows);
    if (b->cols != c->cols)
        return fail(GK_ERR_SHAPE, "gemmkit: B.cols (%zu) != C.cols (%zu)", b->cols, c->cols);
    size_t ea, eb, ec;
    int r;
    if ((r = check_batched_view(a->len, a->rows, a->cols, a->rs, a->cs, batch, a_bs, "A", &ea))) return r;
    if ((r = check_batched_view(b->len, b->rows, b->cols, b->rs, b->cs, batch, b_bs, "B", &eb))) return r;
    if ((r = check_batched_view(c->len, c->rows, c->cols, c->rs, c->cs, batch, c_bs, "C", &ec))) return r;
    if (self_aliases(c->rows, c->cols, c->rs, c->cs))
        return fail(GK_ERR_ALIAS,
                    "gemmkit: batched C element aliases itself (strides %td,%td map distinct "
                    "elements to the same memory); C must address each (i,j) uniquely",
                    c->rs, c->cs);
    if (batch > 1 && (size_t)c_bs < ec)
        return fail(GK_ERR_ALIAS,
                    "gemmkit: C batch stride (%td) must be at least the element extent (%zu) so "
                    "the batched C outputs stay disjoint",
                    c_bs, ec);
    if (overlaps_bytes(c->data, c->len, so, a->data, a->len, si) ||
        overlaps_bytes(c->data, c->len, so, b->data, b->len, si))
        return fail(GK_ERR_ALIAS, "gemmkit: batched C aliases A or B");
    return GK_OK;
}

// ---- fused epilogue selectors (src/api.rs:326-380, src/adapter.rs:130-166)

// Lowers the checked tier's optional bias and activation into `out`, with the
// reference's checks: the bias length matches its axis (m for PerRow, n for
// PerCol), the bias does not overlap C's slice, a LeakyRelu slope is finite.
// `sb`/`so`: bias and C element sizes in bytes.
int lower_fused(const gk_bias *bias, int32_t act, float slope, size_t m, size_t n,
                const gk_mat_mut *c, size_t sb, size_t so, FusedSpec *out) {
    *out = FusedSpec{nullptr, GK_BIAS_PER_ROW, act, slope};
    if (bias) {
        if (bias->dim == GK_BIAS_PER_ROW) {
            if (bias->len != m)
                return fail(GK_ERR_SHAPE, "gemmkit: PerRow bias length (%zu) != A.rows (%zu)",
                            bias->len, m);
        } else if (bias->dim == GK_BIAS_PER_COL) {
            if (bias->len != n)
                return fail(GK_ERR_SHAPE, "gemmkit: PerCol bias length (%zu) != B.cols (%zu)",
                            bias->len, n);
        } else {
            return fail(GK_ERR_ARG, "gemmkit: bias dim (%d) must be 0 (PerRow) or 1 (PerCol)",
                        bias->dim);
        }
        if (overlaps_bytes(c->data, c->len, so, bias->data, bias->len, sb))
            return fail(GK_ERR_ALIAS, "gemmkit: bias slice overlaps C");
        out->bias = bias->data;
        out->dim = bias->dim;
    }
    if (act == GK_ACT_LEAKY_RELU && !std::isfinite(slope))
        return fail(GK_ERR_ARG, "gemmkit: LeakyRelu slope must be finite");
    return GK_OK;
}

int check_act_value(int32_t act) {
    if (act != GK_ACT_NONE && act != GK_ACT_RELU && act != GK_ACT_LEAKY_RELU)
        return fail(GK_ERR_ARG,
                    "gemmkit: activation (%d) must be 0 (none), 1 (Relu) or 2 (LeakyRelu)", act);
    return GK_OK;
}

// ---- prepacked float operands (src/api/packed.rs:67-170, :175-365)

const char *in_name(InType t) {
    return t == InType::I8 ? "i8" : (t == InType::BF16 ? "bf16" : "f32");
}

int check_packed(const gk_packed_rhs *p, InType want) {
    if (!p) return fail(GK_ERR_ARG, "gemmkit: null packed RHS");
    if (p->in != want)
        return fail(GK_ERR_ARG, "gemmkit: packed RHS holds %s elements, this entry takes %s",
                    in_name(p->in), in_name(want));
    return GK_OK;
}

// prepack_rhs_unchecked (src/api/packed.rs:80-170): B^T (n x k) stored
// k-contiguous in an owned device buffer, rows padded to 16 bytes with zeros.
int prepack_any(InType in, const void *b, ptrdiff_t rsb, ptrdiff_t csb, size_t k, size_t n,
                gk_packed_rhs **out) {
    int r;
    if (!out) return fail(GK_ERR_ARG, "gemmkit: null output handle");
    *out = nullptr;
    if ((r = device_init())) return r;
    if (!dims_fit(1, k, n, 1))
        return fail(GK_ERR_OVERFLOW,
                    "gemmkit: prepacked RHS of %zux%zu is too large; the pack buffer size "
                    "overflows usize",
                    k, n);
    const int64_t esz = (int64_t)in_size(in);
    gk_packed_rhs *p = new gk_packed_rhs();
    p->in = in;
    p->k = k;
    p->n = n;
    p->ld = round_up64(std::max<int64_t>((int64_t)k, 1), 16 / esz);
    if (k > 0 && n > 0) {
        size_t bytes = (size_t)p->ld * n * (size_t)esz;
        hipError_t e = hipMalloc(&p->buf, bytes);
        if (e != hipSuccess) {
            delete p;
            return fail(GK_ERR_NOMEM, "gemmkit: prepacked RHS allocation of %zu bytes failed", bytes);
        }
        // Row j of the buffer is column j of B.
        e = launch_pack(in, b, csb, rsb, (int64_t)n, (int64_t)k, p->buf, p->ld, tl_stream);
        if (e == hipSuccess) e = hipStreamSynchronize(tl_stream);
        if (e != hipSuccess) {
            (void)hipFree(p->buf);
            delete p;
            return hip_fail(e, "prepack");
        }
    }
    *out = p;
    return ok();
}

// gemm_packed_b_unchecked's orientation assert (src/api/packed.rs:625-629).
int check_packed_c_layout(ptrdiff_t rsc, ptrdiff_t csc) {
    if ((csc < 0 ? -csc : csc) < (rsc < 0 ? -rsc : rsc))
        return fail(GK_ERR_LAYOUT,
                    "gemmkit: gemm_packed_b requires column-major-ish C (|csc| >= |rsc|); a "
                    "row-major C would swap A/B and invalidate the prepacked RHS \xE2\x80\x94 use "
                    "gemm() for that layout");
    return GK_OK;
}

// gemm_packed_b_with's checks (src/api/packed.rs:191-245): shapes against the
// packed geometry, A and C in bounds, C addresses each element once, C clear
// of A.  `sa`/`so`: A and C element sizes.
int validate_packed_views(const gk_mat_ref *a, const gk_packed_rhs *packed, const gk_mat_mut *c,
                          size_t sa, size_t so) {
    if (!a || !c || !packed) return fail(GK_ERR_ARG, "gemmkit: null argument");
    if (a->cols != packed->k)
        return fail(GK_ERR_SHAPE, "gemmkit: A.cols (%zu) != packed B.rows (%zu)", a->cols, packed->k);
    if (packed->n != c->cols)
        return fail(GK_ERR_SHAPE, "gemmkit: packed B.cols (%zu) != C.cols (%zu)", packed->n, c->cols);
    if (a->rows != c->rows)
        return fail(GK_ERR_SHAPE, "gemmkit: A.rows (%zu) != C.rows (%zu)", a->rows, c->rows);
    int r;
    if ((r = check_view(a->len, a->rows, a->cols, a->rs, a->cs, "A"))) return r;
    if ((r = check_view(c->len, c->rows, c->cols, c->rs, c->cs, "C"))) return r;
    if (self_aliases(c->rows, c->cols, c->rs, c->cs))
        return fail(GK_ERR_ALIAS,
                    "gemmkit: C view aliases itself (strides %td,%td map distinct elements to the "
                    "same memory); C must address each (i,j) uniquely",
                    c->rs, c->cs);
    if (overlaps_bytes(c->data, c->len, so, a->data, a->len, sa))
        return fail(GK_ERR_ALIAS, "gemmkit: C aliases A");
    return GK_OK;
}

// ---- fused / prepacked float entries, shared by the f32 and bf16 ABI twins.
// `in`/`kind`: element type and output epilogue; `esz`: element size; scalars
// already widened to f32.

int fused_checked(gk_workspace *ws, InType in, EpiKind kind, size_t esz, float alpha,
                  const gk_mat_ref *a, const gk_mat_ref *b, float beta, const gk_mat_mut *c,
                  const gk_bias *bias, int32_t act, float slope) {
    int r;
    if ((r = check_act_value(act))) return r;
    if ((r = validate_gemm_views(a, b, c, esz, esz))) return r;
    FusedSpec fx;
    if (bias || act != GK_ACT_NONE) {
        if ((r = lower_fused(bias, act, slope, a->rows, b->cols, c, esz, esz, &fx))) return r;
    }
    // No bias and no activation: the plain GEMM (gemm_fused_with delegates to
    // gemm_with, src/api/fused.rs:93-96).
    return exec_float(ws, in, kind, 1, a->rows, a->cols, b->cols, alpha, a->data, a->rs, a->cs,
                      0, b->data, b->rs, b->cs, 0, beta, c->data, c->rs, c->cs, 0,
                      (bias || act != GK_ACT_NONE) ? &fx : nullptr);
}

int batched_fused_checked(gk_workspace *ws, InType in, EpiKind kind, size_t esz, size_t batch,
                          float alpha, const gk_mat_ref *a, ptrdiff_t a_bs, const gk_mat_ref *b,
                          ptrdiff_t b_bs, float beta, const gk_mat_mut *c, ptrdiff_t c_bs,
                          const gk_bias *bias, int32_t act, float slope) {
    int r;
    if ((r = check_act_value(act))) return r;
    if (batch == 0) return ok();
    if ((r = validate_batched_views(batch, a, a_bs, b, b_bs, c, c_bs, esz, esz))) return r;
    FusedSpec fx;
    const bool any = bias || act != GK_ACT_NONE;
    if (any && (r = lower_fused(bias, act, slope, a->rows, b->cols, c, esz, esz, &fx))) return r;
    return exec_float(ws, in, kind, batch, a->rows, a->cols, b->cols, alpha, a->data, a->rs,
                      a->cs, a_bs, b->data, b->rs, b->cs, b_bs, beta, c->data, c->rs, c->cs, c_bs,
                      any ? &fx : nullptr);
}

int packed_b_unchecked(gk_workspace *ws, InType in, EpiKind kind, float alpha, size_t m,
                       const void *a, ptrdiff_t rsa, ptrdiff_t csa, const gk_packed_rhs *packed,
                       float beta, void *c, ptrdiff_t rsc, ptrdiff_t csc, const FusedSpec *fx) {
    int r;
    if ((r = check_packed(packed, in))) return r;
    if ((r = check_packed_c_layout(rsc, csc))) return r;
    return exec_float(ws, in, kind, 1, m, packed->k, packed->n, alpha, a, rsa, csa, 0, nullptr, 0,
                      0, 0, beta, c, rsc, csc, 0, fx, packed);
}

int packed_b_checked(gk_workspace *ws, InType in, EpiKind kind, size_t esz, float alpha,
                     const gk_mat_ref *a, const gk_packed_rhs *packed, float beta,
                     const gk_mat_mut *c, bool fused, const gk_bias *bias, int32_t act,
                     float slope) {
    int r;
    if (fused && (r = check_act_value(act))) return r;
    if ((r = validate_packed_views(a, packed, c, esz, esz))) return r;
    if ((r = check_packed(packed, in))) return r;
    FusedSpec fx;
    const bool any = fused && (bias || act != GK_ACT_NONE);
    if (any && (r = lower_fused(bias, act, slope, a->rows, packed->n, c, esz, esz, &fx))) return r;
    return packed_b_unchecked(ws, in, kind, alpha, a->rows, a->data, a->rs, a->cs, packed, beta,
                              c->data, c->rs, c->cs, any ? &fx : nullptr);
}

// ---- prepacked LHS (src/api/packed.rs:953-1527)

int check_packed_lhs(const gk_packed_lhs *p, InType want) {
    if (!p) return fail(GK_ERR_ARG, "gemmkit: null packed LHS");
    if (p->in != want)
        return fail(GK_ERR_ARG, "gemmkit: packed LHS holds %s elements, this entry takes %s",
                    in_name(p->in), in_name(want));
    return GK_OK;
}

// prepack_lhs_unchecked (src/api/packed.rs:999-1030): the rows of A stored
// k-contiguous in an owned device buffer, padded to 16 bytes with zeros.  The
// reference packs the transposed product's RHS; its size-overflow message
// names that k x m RHS, and so does this one.
int prepack_lhs_any(InType in, const void *a, ptrdiff_t rsa, ptrdiff_t csa, size_t m, size_t k,
                    gk_packed_lhs **out) {
    int r;
    if (!out) return fail(GK_ERR_ARG, "gemmkit: null output handle");
    *out = nullptr;
    if ((r = device_init())) return r;
    if (!dims_fit(m, k, 1, 1))
        return fail(GK_ERR_OVERFLOW,
                    "gemmkit: prepacked RHS of %zux%zu is too large; the pack buffer size "
                    "overflows usize",
                    k, m);
    const int64_t esz = (int64_t)in_size(in);
    gk_packed_lhs *p = new gk_packed_lhs();
    p->in = in;
    p->m = m;
    p->k = k;
    p->ld = round_up64(std::max<int64_t>((int64_t)k, 1), 16 / esz);
    if (k > 0 && m > 0) {
        size_t bytes = (size_t)p->ld * m * (size_t)esz;
        hipError_t e = hipMalloc(&p->buf, bytes);
        if (e != hipSuccess) {
            delete p;
            return fail(GK_ERR_NOMEM, "gemmkit: prepacked LHS allocation of %zu bytes failed", bytes);
        }
        e = launch_pack(in, a, rsa, csa, (int64_t)m, (int64_t)k, p->buf, p->ld, tl_stream);
        if (e == hipSuccess) e = hipStreamSynchronize(tl_stream);
        if (e != hipSuccess) {
            (void)hipFree(p->buf);
            delete p;
            return hip_fail(e, "prepack");
        }
    }
    *out = p;
    return ok();
}

// gemm_packed_a_unchecked_with's orientation assert (src/api/packed.rs:1190-1194).
int check_packed_a_c_layout(ptrdiff_t rsc, ptrdiff_t csc) {
    if (iabs64(csc) > iabs64(rsc))
        return fail(GK_ERR_LAYOUT,
                    "gemmkit: gemm_packed_a requires row-major-ish C (|csc| <= |rsc|); a "
                    "column-major C would keep A in the LHS role and invalidate the prepacked LHS "
                    "\xE2\x80\x94 use gemm() for that layout");
    return GK_OK;
}

int packed_a_unchecked(gk_workspace *ws, InType in, EpiKind kind, float alpha,
                       const gk_packed_lhs *packed, size_t n, const void *b, ptrdiff_t rsb,
                       ptrdiff_t csb, float beta, void *c, ptrdiff_t rsc, ptrdiff_t csc,
                       const FusedSpec *fx) {
    int r;
    if ((r = check_packed_lhs(packed, in))) return r;
    if ((r = check_packed_a_c_layout(rsc, csc))) return r;
    return exec_float(ws, in, kind, 1, packed->m, packed->k, n, alpha, nullptr, 0, 0, 0, b, rsb,
                      csb, 0, beta, c, rsc, csc, 0, fx, nullptr, packed);
}

// gemm_packed_a_with / gemm_packed_a_fused_with's checks (src/api/packed.rs:1074-1107,
// :1284-1325).
int packed_a_checked(gk_workspace *ws, InType in, EpiKind kind, size_t esz, float alpha,
                     const gk_packed_lhs *packed, const gk_mat_ref *b, float beta,
                     const gk_mat_mut *c, bool fused, const gk_bias *bias, int32_t act,
                     float slope) {
    int r;
    if (fused && (r = check_act_value(act))) return r;
    if (!b || !c || !packed) return fail(GK_ERR_ARG, "gemmkit: null argument");
    if (packed->k != b->rows)
        return fail(GK_ERR_SHAPE, "gemmkit: packed A.cols (%zu) != B.rows (%zu)", packed->k,
                    b->rows);
    if (packed->m != c->rows)
        return fail(GK_ERR_SHAPE, "gemmkit: packed A.rows (%zu) != C.rows (%zu)", packed->m,
                    c->rows);
    if (b->cols != c->cols)
        return fail(GK_ERR_SHAPE, "gemmkit: B.cols (%zu) != C.cols (%zu)", b->cols, c->cols);
    if ((r = check_view(b->len, b->rows, b->cols, b->rs, b->cs, "B"))) return r;
    if ((r = check_view(c->len, c->rows, c->cols, c->rs, c->cs, "C"))) return r;
    if (self_aliases(c->rows, c->cols, c->rs, c->cs))
        return fail(GK_ERR_ALIAS,
                    "gemmkit: C view aliases itself (strides %td,%td map distinct elements to the "
                    "same memory); C must address each (i,j) uniquely",
                    c->rs, c->cs);
    if (overlaps_bytes(c->data, c->len, esz, b->data, b->len, esz))
        return fail(GK_ERR_ALIAS, "gemmkit: C aliases B");
    if ((r = check_packed_lhs(packed, in))) return r;
    FusedSpec fx;
    const bool any = fused && (bias || act != GK_ACT_NONE);
    if (any && (r = lower_fused(bias, act, slope, packed->m, b->cols, c, esz, esz, &fx))) return r;
    return packed_a_unchecked(ws, in, kind, alpha, packed, b->cols, b->data, b->rs, b->cs, beta,
                              c->data, c->rs, c->cs, any ? &fx : nullptr);
}

// ---- pointer-array batched (src/api/batched.rs:711-799; run_ptr,
// src/special/batched.rs:294-334: every problem as a standalone gemm)

// Element step of a run of problems: the pointer difference in elements, when
// it is a whole number of elements.
bool elem_step(const void *p0, const void *p1, size_t esz, ptrdiff_t *step) {
    const ptrdiff_t d = (const char *)p1 - (const char *)p0;
    if (d % (ptrdiff_t)esz) return false;
    *step = d / (ptrdiff_t)esz;
    return true;
}

// Runs problems[0..count) of one element type: runs of consecutive problems
// that share shape, scalars and strides with constant pointer steps go out as
// one strided batched launch (each element bit-identical to the standalone
// product, as gemm_batched's are), the others one by one.
template <typename P, typename S>
int run_problems(gk_workspace *ws, InType in, const P *problems, size_t count, S to_f32) {
    const size_t esz = in_size(in);
    const EpiKind kind = in == InType::F32 ? EpiKind::F32 : EpiKind::BF16;
    size_t i = 0;
    while (i < count) {
        const P &p = problems[i];
        size_t j = i + 1;
        ptrdiff_t sa = 0, sb = 0, sc = 0;
        // (a zero output step would be overlapping outputs, which the caller
        // excludes; such problems run one by one, in order)
        if (j < count && elem_step(p.a, problems[j].a, esz, &sa) &&
            elem_step(p.b, problems[j].b, esz, &sb) && elem_step(p.c, problems[j].c, esz, &sc) &&
            sc != 0) {
            auto same = [&](const P &q, size_t idx) {
                ptrdiff_t qa, qb, qc;
                return q.m == p.m && q.k == p.k && q.n == p.n && q.rsa == p.rsa &&
                       q.csa == p.csa && q.rsb == p.rsb && q.csb == p.csb && q.rsc == p.rsc &&
                       q.csc == p.csc && !memcmp(&q.alpha, &p.alpha, sizeof p.alpha) &&
                       !memcmp(&q.beta, &p.beta, sizeof p.beta) &&
                       elem_step(p.a, q.a, esz, &qa) && qa == sa * (ptrdiff_t)(idx - i) &&
                       elem_step(p.b, q.b, esz, &qb) && qb == sb * (ptrdiff_t)(idx - i) &&
                       elem_step(p.c, q.c, esz, &qc) && qc == sc * (ptrdiff_t)(idx - i);
            };
            while (j < count && same(problems[j], j)) ++j;
        }
        int r;
        if (j - i > 1)
            r = exec_float(ws, in, kind, j - i, p.m, p.k, p.n, to_f32(p.alpha), p.a, p.rsa, p.csa,
                           sa, p.b, p.rsb, p.csb, sb, to_f32(p.beta), p.c, p.rsc, p.csc, sc);
        else
            r = exec_float(ws, in, kind, 1, p.m, p.k, p.n, to_f32(p.alpha), p.a, p.rsa, p.csa, 0,
                           p.b, p.rsb, p.csb, 0, to_f32(p.beta), p.c, p.rsc, p.csc, 0);
        if (r) return r;
        i = j;
    }
    return ok();
}

// gemm_batched_slice's per-element checks (src/api/batched.rs:751-783).
int validate_batch_problem(size_t i, const gk_mat_ref &a, const gk_mat_ref &b,
                           const gk_mat_mut &c) {
    if (a.cols != b.rows)
        return fail(GK_ERR_SHAPE, "gemmkit: batch element %zu A.cols (%zu) != B.rows (%zu)", i,
                    a.cols, b.rows);
    if (a.rows != c.rows)
        return fail(GK_ERR_SHAPE, "gemmkit: batch element %zu A.rows (%zu) != C.rows (%zu)", i,
                    a.rows, c.rows);
    if (b.cols != c.cols)
        return fail(GK_ERR_SHAPE, "gemmkit: batch element %zu B.cols (%zu) != C.cols (%zu)", i,
                    b.cols, c.cols);
    int r;
    if ((r = check_view(a.len, a.rows, a.cols, a.rs, a.cs, "A"))) return r;
    if ((r = check_view(b.len, b.rows, b.cols, b.rs, b.cs, "B"))) return r;
    if ((r = check_view(c.len, c.rows, c.cols, c.rs, c.cs, "C"))) return r;
    if (self_aliases(c.rows, c.cols, c.rs, c.cs))
        return fail(GK_ERR_ALIAS,
                    "gemmkit: batch element %zu C view aliases itself (strides %td,%td); C must "
                    "address each (i,j) uniquely",
                    i, c.rs, c.cs);
    return GK_OK;
}

template <typename BP, typename P, typename S>
int batched_slice(gk_workspace *ws, const BP *problems, size_t count, gk_par par,
                  int (*run)(gk_workspace *, const P *, size_t, gk_par)) {
    if (count == 0) return ok();
    if (!problems) return fail(GK_ERR_ARG, "gemmkit: null problems array");
    std::vector<P> raw(count);
    for (size_t i = 0; i < count; ++i) {
        const BP &q = problems[i];
        int r = validate_batch_problem(i, q.a, q.b, q.c);
        if (r) return r;
        raw[i] = P{q.a.rows, q.a.cols, q.b.cols, q.alpha, (const S *)q.a.data, q.a.rs, q.a.cs,
                   (const S *)q.b.data, q.b.rs, q.b.cs, q.beta, (S *)q.c.data, q.c.rs, q.c.cs};
    }
    return run(ws, raw.data(), count, par);
}

}  // namespace

// =============================================================== C ABI

extern "C" {

const char *gk_last_error(void) { return tl_error.c_str(); }

const char *gk_version(void) { return "gemmkit-hip 0.1.0 (gfx950)"; }

int gk_debug_plan(int32_t in, int32_t kind, int64_t m, int64_t n, int64_t batch, int64_t kbytes,
                  int64_t ld_b, int32_t *tile, int64_t *na, int32_t *tile_b, int32_t *pn_a,
                  int32_t *pn_b) {
    if (in < 0 || in > 2 || kind < 0 || kind > 3 || m <= 0 || n <= 0 || batch <= 0 ||
        kbytes < 0 || ld_b < 0 || !tile || !na || !tile_b)
        return fail(GK_ERR_ARG, "gemmkit: gk_debug_plan: bad argument");
    if (ld_b == 0) ld_b = (kbytes + 15) / 16 * 16;
    const MmaPlan plan = plan_mma(m, n, batch, kbytes, (EpiKind)kind, (InType)in, ld_b);
    *tile = (int32_t)plan.ta;
    *na = plan.na < n ? plan.na : 0;
    *tile_b = (int32_t)plan.tb;
    if (pn_a) *pn_a = plan.pn_a;
    if (pn_b) *pn_b = plan.pn_b;
    return ok();
}

int gk_init(void) {
    int r = device_init();
    return r ? r : ok();
}

int gk_set_stream(void *hip_stream) {
    tl_stream = (hipStream_t)hip_stream;
    return ok();
}

void *gk_get_stream(void) { return (void *)tl_stream; }

int gk_set_synchronous(int on) {
    tl_sync = on ? 1 : 0;
    return ok();
}

gk_workspace *gk_workspace_new(void) { return new gk_workspace(); }

gk_workspace *gk_workspace_with_capacity(size_t bytes) {
    gk_workspace *ws = new gk_workspace();
    if (bytes > 0) {
        void *p = nullptr;
        if (device_init() || ws_reserve(ws, bytes, &p)) {
            delete ws;
            return nullptr;
        }
    }
    return ws;
}

void gk_workspace_free(gk_workspace *ws) {
    if (!ws) return;
    ws_release(ws);
    delete ws;
}

size_t gk_workspace_bytes(const gk_workspace *ws) { return ws ? ws->bytes : 0; }

// ---- f32

int gk_gemm_f32_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, float alpha,
                          const float *a, ptrdiff_t rsa, ptrdiff_t csa, const float *b,
                          ptrdiff_t rsb, ptrdiff_t csb, float beta, float *c, ptrdiff_t rsc,
                          ptrdiff_t csc, gk_par) {
    return exec_float(ws, InType::F32, EpiKind::F32, 1, m, k, n, alpha, a, rsa, csa, 0, b, rsb,
                      csb, 0, beta, c, rsc, csc, 0);
}

int gk_gemm_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                float beta, const gk_mat_mut *c, gk_par par) {
    int r = validate_gemm_views(a, b, c, 4, 4);
    if (r) return r;
    return gk_gemm_f32_unchecked(ws, a->rows, a->cols, b->cols, alpha, (const float *)a->data,
                                 a->rs, a->cs, (const float *)b->data, b->rs, b->cs, beta,
                                 (float *)c->data, c->rs, c->cs, par);
}

// ---- bf16

int gk_gemm_bf16_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, gk_bf16 alpha,
                           const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa, const gk_bf16 *b,
                           ptrdiff_t rsb, ptrdiff_t csb, gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc,
                           ptrdiff_t csc, gk_par) {
    return exec_float(ws, InType::BF16, EpiKind::BF16, 1, m, k, n, bf16_to_f32(alpha), a, rsa,
                      csa, 0, b, rsb, csb, 0, bf16_to_f32(beta), c, rsc, csc, 0);
}

int gk_gemm_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                 gk_bf16 beta, const gk_mat_mut *c, gk_par par) {
    int r = validate_gemm_views(a, b, c, 2, 2);
    if (r) return r;
    return gk_gemm_bf16_unchecked(ws, a->rows, a->cols, b->cols, alpha, (const gk_bf16 *)a->data,
                                  a->rs, a->cs, (const gk_bf16 *)b->data, b->rs, b->cs, beta,
                                  (gk_bf16 *)c->data, c->rs, c->cs, par);
}

int gk_gemm_bf16_f32out_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, float alpha,
                                  const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                  const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb, float beta,
                                  float *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par) {
    return exec_float(ws, InType::BF16, EpiKind::F32, 1, m, k, n, alpha, a, rsa, csa, 0, b, rsb,
                      csb, 0, beta, c, rsc, csc, 0);
}

int gk_gemm_bf16_f32out(gk_workspace *ws, float alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                        float beta, const gk_mat_mut *c, gk_par par) {
    int r = validate_gemm_views(a, b, c, 2, 4);
    if (r) return r;
    return gk_gemm_bf16_f32out_unchecked(ws, a->rows, a->cols, b->cols, alpha,
                                         (const gk_bf16 *)a->data, a->rs, a->cs,
                                         (const gk_bf16 *)b->data, b->rs, b->cs, beta,
                                         (float *)c->data, c->rs, c->cs, par);
}

// ---- i8

int gk_gemm_i8_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, int32_t alpha,
                         const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa, const int8_t *b,
                         ptrdiff_t rsb, ptrdiff_t csb, int32_t beta, int32_t *c, ptrdiff_t rsc,
                         ptrdiff_t csc, gk_par) {
    return exec_i8(ws, m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc);
}

// The no-allocation twin of gk_gemm_i8_unchecked: the same route and kernels,
// with the static per-device scratch in place of the workspace arena.  Calls
// that overlap on one device share that scratch and race.
int gk_gemm_i8_unchecked_noalloc(size_t m, size_t k, size_t n, int32_t alpha, const int8_t *a,
                                 ptrdiff_t rsa, ptrdiff_t csa, const int8_t *b, ptrdiff_t rsb,
                                 ptrdiff_t csb, int32_t beta, int32_t *c, ptrdiff_t rsc,
                                 ptrdiff_t csc, gk_par) {
    int r;
    if ((r = device_init())) return r;
    uint8_t *sp = nullptr;
    if ((r = scratch_for_current_device(&sp))) return r;
    const Region rg{nullptr, sp, kNoAllocScratchBytes};
    return exec_i8(nullptr, m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc, nullptr,
                   &rg);
}

int gk_gemm_i8(gk_workspace *ws, int32_t alpha, const gk_mat_ref *a, const gk_mat_ref *b,
               int32_t beta, const gk_mat_mut *c, gk_par par) {
    int r = validate_gemm_views(a, b, c, 1, 4);
    if (r) return r;
    return gk_gemm_i8_unchecked(ws, a->rows, a->cols, b->cols, alpha, (const int8_t *)a->data,
                                a->rs, a->cs, (const int8_t *)b->data, b->rs, b->cs, beta,
                                (int32_t *)c->data, c->rs, c->cs, par);
}

// ---- requant

int gk_gemm_i8_requant(gk_workspace *ws, const gk_mat_ref *a, const gk_mat_ref *b,
                       const gk_requantize *req, const gk_mat_mut *c, gk_par) {
    return requant_checked(ws, a, b, nullptr, req, c, false);
}

int gk_gemm_i8_requant_u8(gk_workspace *ws, const gk_mat_ref *a, const gk_mat_ref *b,
                          const gk_requantize *req, const gk_mat_mut *c, gk_par) {
    return requant_checked(ws, a, b, nullptr, req, c, true);
}

int gk_gemm_i8_requant_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, const int8_t *a,
                                 ptrdiff_t rsa, ptrdiff_t csa, const int8_t *b, ptrdiff_t rsb,
                                 ptrdiff_t csb, float scale, const float *row_scales,
                                 uint8_t has_row_scales, int32_t zero_point, const int32_t *bias,
                                 uint8_t has_bias, int8_t *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par,
                                 int32_t axis, int32_t act) {
    return exec_requant(ws, m, k, n, a, rsa, csa, b, rsb, csb, scale,
                        has_row_scales ? row_scales : nullptr, zero_point,
                        has_bias ? bias : nullptr, axis, act, -128, 127, c, rsc, csc);
}

int gk_gemm_i8_requant_u8_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n,
                                    const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                                    const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb, float scale,
                                    const float *row_scales, uint8_t has_row_scales,
                                    int32_t zero_point, const int32_t *bias, uint8_t has_bias,
                                    uint8_t *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par, int32_t axis,
                                    int32_t act) {
    return exec_requant(ws, m, k, n, a, rsa, csa, b, rsb, csb, scale,
                        has_row_scales ? row_scales : nullptr, zero_point,
                        has_bias ? bias : nullptr, axis, act, 0, 255, c, rsc, csc);
}

// ---- prepacked RHS (src/api/packed.rs:372-656)

int gk_prepack_rhs_i8_unchecked(const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb, size_t k, size_t n,
                                gk_packed_rhs **out) {
    return prepack_any(InType::I8, b, rsb, csb, k, n, out);
}

int gk_prepack_rhs_i8(const gk_mat_ref *b, gk_packed_rhs **out) {
    if (!b) return fail(GK_ERR_ARG, "gemmkit: null view argument");
    int r = check_view(b->len, b->rows, b->cols, b->rs, b->cs, "B");
    if (r) return r;
    return gk_prepack_rhs_i8_unchecked((const int8_t *)b->data, b->rs, b->cs, b->rows, b->cols, out);
}

int gk_prepack_rhs_f32_unchecked(const float *b, ptrdiff_t rsb, ptrdiff_t csb, size_t k, size_t n,
                                 gk_packed_rhs **out) {
    return prepack_any(InType::F32, b, rsb, csb, k, n, out);
}

int gk_prepack_rhs_f32(const gk_mat_ref *b, gk_packed_rhs **out) {
    if (!b) return fail(GK_ERR_ARG, "gemmkit: null view argument");
    int r = check_view(b->len, b->rows, b->cols, b->rs, b->cs, "B");
    if (r) return r;
    return prepack_any(InType::F32, b->data, b->rs, b->cs, b->rows, b->cols, out);
}

int gk_prepack_rhs_bf16_unchecked(const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb, size_t k,
                                  size_t n, gk_packed_rhs **out) {
    return prepack_any(InType::BF16, b, rsb, csb, k, n, out);
}

int gk_prepack_rhs_bf16(const gk_mat_ref *b, gk_packed_rhs **out) {
    if (!b) return fail(GK_ERR_ARG, "gemmkit: null view argument");
    int r = check_view(b->len, b->rows, b->cols, b->rs, b->cs, "B");
    if (r) return r;
    return prepack_any(InType::BF16, b->data, b->rs, b->cs, b->rows, b->cols, out);
}

void gk_packed_rhs_free(gk_packed_rhs *p) {
    if (!p) return;
    if (p->buf) {
        (void)hipDeviceSynchronize();
        (void)hipFree(p->buf);
    }
    delete p;
}

size_t gk_packed_rhs_rows(const gk_packed_rhs *p) { return p ? p->k : 0; }
size_t gk_packed_rhs_cols(const gk_packed_rhs *p) { return p ? p->n : 0; }

int gk_gemm_i8_packed_b_unchecked(gk_workspace *ws, int32_t alpha, size_t m, const int8_t *a,
                                  ptrdiff_t rsa, ptrdiff_t csa, const gk_packed_rhs *packed,
                                  int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par) {
    int r;
    if ((r = check_packed(packed, InType::I8))) return r;
    if ((r = check_packed_c_layout(rsc, csc))) return r;
    return exec_i8(ws, m, packed->k, packed->n, alpha, a, rsa, csa, nullptr, 0, 0, beta, c, rsc,
                   csc, packed);
}

int gk_gemm_i8_packed_b(gk_workspace *ws, int32_t alpha, const gk_mat_ref *a,
                        const gk_packed_rhs *packed, int32_t beta, const gk_mat_mut *c,
                        gk_par par) {
    int r;
    if ((r = validate_packed_views(a, packed, c, 1, 4))) return r;
    if ((r = check_packed(packed, InType::I8))) return r;
    return gk_gemm_i8_packed_b_unchecked(ws, alpha, a->rows, (const int8_t *)a->data, a->rs, a->cs,
                                         packed, beta, (int32_t *)c->data, c->rs, c->cs, par);
}

int gk_gemm_i8_packed_b_requant(gk_workspace *ws, const gk_mat_ref *a, const gk_packed_rhs *packed,
                                const gk_requantize *req, const gk_mat_mut *c, gk_par) {
    if (int r = check_packed(packed, InType::I8)) return r;
    return requant_checked(ws, a, nullptr, packed, req, c, false);
}

int gk_gemm_i8_packed_b_requant_u8(gk_workspace *ws, const gk_mat_ref *a,
                                   const gk_packed_rhs *packed, const gk_requantize *req,
                                   const gk_mat_mut *c, gk_par) {
    if (int r = check_packed(packed, InType::I8)) return r;
    return requant_checked(ws, a, nullptr, packed, req, c, true);
}

int gk_gemm_i8_packed_b_requant_unchecked(gk_workspace *ws, size_t m, const int8_t *a,
                                          ptrdiff_t rsa, ptrdiff_t csa,
                                          const gk_packed_rhs *packed, float scale,
                                          const float *scales, uint8_t has_scales,
                                          int32_t zero_point, const int32_t *bias,
                                          uint8_t has_bias, int8_t *c, ptrdiff_t rsc,
                                          ptrdiff_t csc, gk_par, int32_t axis, int32_t act) {
    if (int r = check_packed(packed, InType::I8)) return r;
    return exec_requant(ws, m, packed->k, packed->n, a, rsa, csa, nullptr, 0, 0, scale,
                        has_scales ? scales : nullptr, zero_point, has_bias ? bias : nullptr, axis,
                        act, -128, 127, c, rsc, csc, packed);
}

int gk_gemm_i8_packed_b_requant_u8_unchecked(gk_workspace *ws, size_t m, const int8_t *a,
                                             ptrdiff_t rsa, ptrdiff_t csa,
                                             const gk_packed_rhs *packed, float scale,
                                             const float *scales, uint8_t has_scales,
                                             int32_t zero_point, const int32_t *bias,
                                             uint8_t has_bias, uint8_t *c, ptrdiff_t rsc,
                                             ptrdiff_t csc, gk_par, int32_t axis, int32_t act) {
    if (int r = check_packed(packed, InType::I8)) return r;
    return exec_requant(ws, m, packed->k, packed->n, a, rsa, csa, nullptr, 0, 0, scale,
                        has_scales ? scales : nullptr, zero_point, has_bias ? bias : nullptr, axis,
                        act, 0, 255, c, rsc, csc, packed);
}

// ---- batched (src/api/batched.rs:188-711)

int gk_gemm_batched_f32_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k, size_t n,
                                  float alpha, const float *a, ptrdiff_t rsa, ptrdiff_t csa,
                                  ptrdiff_t a_bs, const float *b, ptrdiff_t rsb, ptrdiff_t csb,
                                  ptrdiff_t b_bs, float beta, float *c, ptrdiff_t rsc,
                                  ptrdiff_t csc, ptrdiff_t c_bs, gk_par) {
    return exec_float(ws, InType::F32, EpiKind::F32, batch, m, k, n, alpha, a, rsa, csa, a_bs, b,
                      rsb, csb, b_bs, beta, c, rsc, csc, c_bs);
}

int gk_gemm_batched_f32(gk_workspace *ws, size_t batch, float alpha, const gk_mat_ref *a,
                        ptrdiff_t a_bs, const gk_mat_ref *b, ptrdiff_t b_bs, float beta,
                        const gk_mat_mut *c, ptrdiff_t c_bs, gk_par par) {
    if (batch == 0) return ok();
    int r = validate_batched_views(batch, a, a_bs, b, b_bs, c, c_bs, 4, 4);
    if (r) return r;
    return gk_gemm_batched_f32_unchecked(ws, batch, a->rows, a->cols, b->cols, alpha,
                                         (const float *)a->data, a->rs, a->cs, a_bs,
                                         (const float *)b->data, b->rs, b->cs, b_bs, beta,
                                         (float *)c->data, c->rs, c->cs, c_bs, par);
}

int gk_gemm_batched_bf16_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k, size_t n,
                                   gk_bf16 alpha, const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                   ptrdiff_t a_bs, const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                                   ptrdiff_t b_bs, gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc,
                                   ptrdiff_t csc, ptrdiff_t c_bs, gk_par) {
    return exec_float(ws, InType::BF16, EpiKind::BF16, batch, m, k, n, bf16_to_f32(alpha), a, rsa,
                      csa, a_bs, b, rsb, csb, b_bs, bf16_to_f32(beta), c, rsc, csc, c_bs);
}

int gk_gemm_batched_bf16(gk_workspace *ws, size_t batch, gk_bf16 alpha, const gk_mat_ref *a,
                         ptrdiff_t a_bs, const gk_mat_ref *b, ptrdiff_t b_bs, gk_bf16 beta,
                         const gk_mat_mut *c, ptrdiff_t c_bs, gk_par par) {
    if (batch == 0) return ok();
    int r = validate_batched_views(batch, a, a_bs, b, b_bs, c, c_bs, 2, 2);
    if (r) return r;
    return gk_gemm_batched_bf16_unchecked(ws, batch, a->rows, a->cols, b->cols, alpha,
                                          (const gk_bf16 *)a->data, a->rs, a->cs, a_bs,
                                          (const gk_bf16 *)b->data, b->rs, b->cs, b_bs, beta,
                                          (gk_bf16 *)c->data, c->rs, c->cs, c_bs, par);
}

int gk_gemm_batched_ptr_f32_unchecked(gk_workspace *ws, const gk_problem_f32 *problems,
                                      size_t count, gk_par) {
    if (count == 0) return ok();
    if (!problems) return fail(GK_ERR_ARG, "gemmkit: null problems array");
    return run_problems(ws, InType::F32, problems, count, [](float v) { return v; });
}

int gk_gemm_batched_ptr_bf16_unchecked(gk_workspace *ws, const gk_problem_bf16 *problems,
                                       size_t count, gk_par) {
    if (count == 0) return ok();
    if (!problems) return fail(GK_ERR_ARG, "gemmkit: null problems array");
    return run_problems(ws, InType::BF16, problems, count,
                        [](gk_bf16 v) { return bf16_to_f32(v); });
}

int gk_gemm_batched_slice_f32(gk_workspace *ws, const gk_batch_problem_f32 *problems,
                              size_t count, gk_par par) {
    return batched_slice<gk_batch_problem_f32, gk_problem_f32, float>(
        ws, problems, count, par, gk_gemm_batched_ptr_f32_unchecked);
}

int gk_gemm_batched_slice_bf16(gk_workspace *ws, const gk_batch_problem_bf16 *problems,
                               size_t count, gk_par par) {
    return batched_slice<gk_batch_problem_bf16, gk_problem_bf16, gk_bf16>(
        ws, problems, count, par, gk_gemm_batched_ptr_bf16_unchecked);
}

int gk_gemm_batched_bf16_f32out_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                          size_t n, float alpha, const gk_bf16 *a, ptrdiff_t rsa,
                                          ptrdiff_t csa, ptrdiff_t a_bs, const gk_bf16 *b,
                                          ptrdiff_t rsb, ptrdiff_t csb, ptrdiff_t b_bs, float beta,
                                          float *c, ptrdiff_t rsc, ptrdiff_t csc, ptrdiff_t c_bs,
                                          gk_par) {
    return exec_float(ws, InType::BF16, EpiKind::F32, batch, m, k, n, alpha, a, rsa, csa, a_bs, b,
                      rsb, csb, b_bs, beta, c, rsc, csc, c_bs);
}

int gk_gemm_batched_bf16_f32out(gk_workspace *ws, size_t batch, float alpha, const gk_mat_ref *a,
                                ptrdiff_t a_bs, const gk_mat_ref *b, ptrdiff_t b_bs, float beta,
                                const gk_mat_mut *c, ptrdiff_t c_bs, gk_par par) {
    if (batch == 0) return ok();
    int r = validate_batched_views(batch, a, a_bs, b, b_bs, c, c_bs, 2, 4);
    if (r) return r;
    return gk_gemm_batched_bf16_f32out_unchecked(ws, batch, a->rows, a->cols, b->cols, alpha,
                                                 (const gk_bf16 *)a->data, a->rs, a->cs, a_bs,
                                                 (const gk_bf16 *)b->data, b->rs, b->cs, b_bs,
                                                 beta, (float *)c->data, c->rs, c->cs, c_bs, par);
}

// ---- prepacked float RHS (src/api/packed.rs:175-365)

int gk_gemm_packed_b_f32_unchecked(gk_workspace *ws, float alpha, size_t m, const float *a,
                                   ptrdiff_t rsa, ptrdiff_t csa, const gk_packed_rhs *packed,
                                   float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par) {
    return packed_b_unchecked(ws, InType::F32, EpiKind::F32, alpha, m, a, rsa, csa, packed, beta,
                              c, rsc, csc, nullptr);
}

int gk_gemm_packed_b_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a,
                         const gk_packed_rhs *packed, float beta, const gk_mat_mut *c, gk_par) {
    return packed_b_checked(ws, InType::F32, EpiKind::F32, 4, alpha, a, packed, beta, c, false,
                            nullptr, GK_ACT_NONE, 0.0f);
}

int gk_gemm_packed_b_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha, size_t m, const gk_bf16 *a,
                                    ptrdiff_t rsa, ptrdiff_t csa, const gk_packed_rhs *packed,
                                    gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                    gk_par) {
    return packed_b_unchecked(ws, InType::BF16, EpiKind::BF16, bf16_to_f32(alpha), m, a, rsa, csa,
                              packed, bf16_to_f32(beta), c, rsc, csc, nullptr);
}

int gk_gemm_packed_b_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a,
                          const gk_packed_rhs *packed, gk_bf16 beta, const gk_mat_mut *c, gk_par) {
    return packed_b_checked(ws, InType::BF16, EpiKind::BF16, 2, bf16_to_f32(alpha), a, packed,
                            bf16_to_f32(beta), c, false, nullptr, GK_ACT_NONE, 0.0f);
}

// ---- prepacked LHS (src/api/packed.rs:953-1527)

int gk_prepack_lhs_f32_unchecked(const float *a, ptrdiff_t rsa, ptrdiff_t csa, size_t m, size_t k,
                                 gk_packed_lhs **out) {
    return prepack_lhs_any(InType::F32, a, rsa, csa, m, k, out);
}

int gk_prepack_lhs_f32(const gk_mat_ref *a, gk_packed_lhs **out) {
    if (!a) return fail(GK_ERR_ARG, "gemmkit: null view argument");
    int r = check_view(a->len, a->rows, a->cols, a->rs, a->cs, "A");
    if (r) return r;
    return prepack_lhs_any(InType::F32, a->data, a->rs, a->cs, a->rows, a->cols, out);
}

int gk_prepack_lhs_bf16_unchecked(const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa, size_t m,
                                  size_t k, gk_packed_lhs **out) {
    return prepack_lhs_any(InType::BF16, a, rsa, csa, m, k, out);
}

int gk_prepack_lhs_bf16(const gk_mat_ref *a, gk_packed_lhs **out) {
    if (!a) return fail(GK_ERR_ARG, "gemmkit: null view argument");
    int r = check_view(a->len, a->rows, a->cols, a->rs, a->cs, "A");
    if (r) return r;
    return prepack_lhs_any(InType::BF16, a->data, a->rs, a->cs, a->rows, a->cols, out);
}

void gk_packed_lhs_free(gk_packed_lhs *p) {
    if (!p) return;
    if (p->buf) {
        (void)hipDeviceSynchronize();
        (void)hipFree(p->buf);
    }
    delete p;
}

size_t gk_packed_lhs_rows(const gk_packed_lhs *p) { return p ? p->m : 0; }
size_t gk_packed_lhs_cols(const gk_packed_lhs *p) { return p ? p->k : 0; }

int gk_gemm_packed_a_f32_unchecked(gk_workspace *ws, float alpha, const gk_packed_lhs *packed,
                                   size_t n, const float *b, ptrdiff_t rsb, ptrdiff_t csb,
                                   float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par) {
    return packed_a_unchecked(ws, InType::F32, EpiKind::F32, alpha, packed, n, b, rsb, csb, beta,
                              c, rsc, csc, nullptr);
}

int gk_gemm_packed_a_f32(gk_workspace *ws, float alpha, const gk_packed_lhs *packed,
                         const gk_mat_ref *b, float beta, const gk_mat_mut *c, gk_par) {
    return packed_a_checked(ws, InType::F32, EpiKind::F32, 4, alpha, packed, b, beta, c, false,
                            nullptr, GK_ACT_NONE, 0.0f);
}

int gk_gemm_packed_a_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha, const gk_packed_lhs *packed,
                                    size_t n, const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                                    gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                    gk_par) {
    return packed_a_unchecked(ws, InType::BF16, EpiKind::BF16, bf16_to_f32(alpha), packed, n, b,
                              rsb, csb, bf16_to_f32(beta), c, rsc, csc, nullptr);
}

int gk_gemm_packed_a_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_packed_lhs *packed,
                          const gk_mat_ref *b, gk_bf16 beta, const gk_mat_mut *c, gk_par) {
    return packed_a_checked(ws, InType::BF16, EpiKind::BF16, 2, bf16_to_f32(alpha), packed, b,
                            bf16_to_f32(beta), c, false, nullptr, GK_ACT_NONE, 0.0f);
}

int gk_gemm_packed_a_fused_f32(gk_workspace *ws, float alpha, const gk_packed_lhs *packed,
                               const gk_mat_ref *b, float beta, const gk_mat_mut *c,
                               const gk_bias *bias, int32_t act, float slope, gk_par) {
    return packed_a_checked(ws, InType::F32, EpiKind::F32, 4, alpha, packed, b, beta, c, true,
                            bias, act, slope);
}

int gk_gemm_packed_a_fused_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_packed_lhs *packed,
                                const gk_mat_ref *b, gk_bf16 beta, const gk_mat_mut *c,
                                const gk_bias *bias, int32_t act, gk_bf16 slope, gk_par) {
    return packed_a_checked(ws, InType::BF16, EpiKind::BF16, 2, bf16_to_f32(alpha), packed, b,
                            bf16_to_f32(beta), c, true, bias, act, bf16_to_f32(slope));
}

int gk_gemm_packed_a_fused_f32_unchecked(gk_workspace *ws, float alpha,
                                         const gk_packed_lhs *packed, size_t n, const float *b,
                                         ptrdiff_t rsb, ptrdiff_t csb, float beta, float *c,
                                         ptrdiff_t rsc, ptrdiff_t csc, const float *bias,
                                         int32_t bias_dim, uint8_t has_bias, int32_t act,
                                         float slope, gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, slope};
    return packed_a_unchecked(ws, InType::F32, EpiKind::F32, alpha, packed, n, b, rsb, csb, beta,
                              c, rsc, csc, &fx);
}

int gk_gemm_packed_a_fused_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha,
                                          const gk_packed_lhs *packed, size_t n,
                                          const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                                          gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                          const gk_bf16 *bias, int32_t bias_dim,
                                          uint8_t has_bias, int32_t act, gk_bf16 slope, gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, bf16_to_f32(slope)};
    return packed_a_unchecked(ws, InType::BF16, EpiKind::BF16, bf16_to_f32(alpha), packed, n, b,
                              rsb, csb, bf16_to_f32(beta), c, rsc, csc, &fx);
}

// ---- fused bias / activation (src/api/fused.rs, src/api/batched.rs:307-590,
// src/api/packed.rs:684-950)

int gk_gemm_fused_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                      float beta, const gk_mat_mut *c, const gk_bias *bias, int32_t act,
                      float slope, gk_par) {
    return fused_checked(ws, InType::F32, EpiKind::F32, 4, alpha, a, b, beta, c, bias, act, slope);
}

int gk_gemm_fused_f32_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, float alpha,
                                const float *a, ptrdiff_t rsa, ptrdiff_t csa, const float *b,
                                ptrdiff_t rsb, ptrdiff_t csb, float beta, float *c, ptrdiff_t rsc,
                                ptrdiff_t csc, const float *bias, int32_t bias_dim,
                                uint8_t has_bias, int32_t act, float slope, gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, slope};
    return exec_float(ws, InType::F32, EpiKind::F32, 1, m, k, n, alpha, a, rsa, csa, 0, b, rsb,
                      csb, 0, beta, c, rsc, csc, 0, &fx);
}

int gk_gemm_fused_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                       gk_bf16 beta, const gk_mat_mut *c, const gk_bias *bias, int32_t act,
                       gk_bf16 slope, gk_par) {
    return fused_checked(ws, InType::BF16, EpiKind::BF16, 2, bf16_to_f32(alpha), a, b,
                         bf16_to_f32(beta), c, bias, act, bf16_to_f32(slope));
}

int gk_gemm_fused_bf16_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, gk_bf16 alpha,
                                 const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa, const gk_bf16 *b,
                                 ptrdiff_t rsb, ptrdiff_t csb, gk_bf16 beta, gk_bf16 *c,
                                 ptrdiff_t rsc, ptrdiff_t csc, const gk_bf16 *bias,
                                 int32_t bias_dim, uint8_t has_bias, int32_t act, gk_bf16 slope,
                                 gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, bf16_to_f32(slope)};
    return exec_float(ws, InType::BF16, EpiKind::BF16, 1, m, k, n, bf16_to_f32(alpha), a, rsa, csa,
                      0, b, rsb, csb, 0, bf16_to_f32(beta), c, rsc, csc, 0, &fx);
}

int gk_gemm_batched_fused_f32(gk_workspace *ws, size_t batch, float alpha, const gk_mat_ref *a,
                              ptrdiff_t a_bs, const gk_mat_ref *b, ptrdiff_t b_bs, float beta,
                              const gk_mat_mut *c, ptrdiff_t c_bs, const gk_bias *bias,
                              int32_t act, float slope, gk_par) {
    return batched_fused_checked(ws, InType::F32, EpiKind::F32, 4, batch, alpha, a, a_bs, b, b_bs,
                                 beta, c, c_bs, bias, act, slope);
}

int gk_gemm_batched_fused_f32_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                        size_t n, float alpha, const float *a, ptrdiff_t rsa,
                                        ptrdiff_t csa, ptrdiff_t a_bs, const float *b,
                                        ptrdiff_t rsb, ptrdiff_t csb, ptrdiff_t b_bs, float beta,
                                        float *c, ptrdiff_t rsc, ptrdiff_t csc, ptrdiff_t c_bs,
                                        const float *bias, int32_t bias_dim, uint8_t has_bias,
                                        int32_t act, float slope, gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, slope};
    return exec_float(ws, InType::F32, EpiKind::F32, batch, m, k, n, alpha, a, rsa, csa, a_bs, b,
                      rsb, csb, b_bs, beta, c, rsc, csc, c_bs, &fx);
}

int gk_gemm_batched_fused_bf16(gk_workspace *ws, size_t batch, gk_bf16 alpha,
                               const gk_mat_ref *a, ptrdiff_t a_bs, const gk_mat_ref *b,
                               ptrdiff_t b_bs, gk_bf16 beta, const gk_mat_mut *c, ptrdiff_t c_bs,
                               const gk_bias *bias, int32_t act, gk_bf16 slope, gk_par) {
    return batched_fused_checked(ws, InType::BF16, EpiKind::BF16, 2, batch, bf16_to_f32(alpha), a,
                                 a_bs, b, b_bs, bf16_to_f32(beta), c, c_bs, bias, act,
                                 bf16_to_f32(slope));
}

int gk_gemm_batched_fused_bf16_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                         size_t n, gk_bf16 alpha, const gk_bf16 *a, ptrdiff_t rsa,
                                         ptrdiff_t csa, ptrdiff_t a_bs, const gk_bf16 *b,
                                         ptrdiff_t rsb, ptrdiff_t csb, ptrdiff_t b_bs,
                                         gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                         ptrdiff_t c_bs, const gk_bf16 *bias, int32_t bias_dim,
                                         uint8_t has_bias, int32_t act, gk_bf16 slope, gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, bf16_to_f32(slope)};
    return exec_float(ws, InType::BF16, EpiKind::BF16, batch, m, k, n, bf16_to_f32(alpha), a, rsa,
                      csa, a_bs, b, rsb, csb, b_bs, bf16_to_f32(beta), c, rsc, csc, c_bs, &fx);
}

int gk_gemm_packed_b_fused_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a,
                               const gk_packed_rhs *packed, float beta, const gk_mat_mut *c,
                               const gk_bias *bias, int32_t act, float slope, gk_par) {
    return packed_b_checked(ws, InType::F32, EpiKind::F32, 4, alpha, a, packed, beta, c, true,
                            bias, act, slope);
}

int gk_gemm_packed_b_fused_f32_unchecked(gk_workspace *ws, float alpha, size_t m, const float *a,
                                         ptrdiff_t rsa, ptrdiff_t csa,
                                         const gk_packed_rhs *packed, float beta, float *c,
                                         ptrdiff_t rsc, ptrdiff_t csc, const float *bias,
                                         int32_t bias_dim, uint8_t has_bias, int32_t act,
                                         float slope, gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, slope};
    return packed_b_unchecked(ws, InType::F32, EpiKind::F32, alpha, m, a, rsa, csa, packed, beta,
                              c, rsc, csc, &fx);
}

int gk_gemm_packed_b_fused_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a,
                                const gk_packed_rhs *packed, gk_bf16 beta, const gk_mat_mut *c,
                                const gk_bias *bias, int32_t act, gk_bf16 slope, gk_par) {
    return packed_b_checked(ws, InType::BF16, EpiKind::BF16, 2, bf16_to_f32(alpha), a, packed,
                            bf16_to_f32(beta), c, true, bias, act, bf16_to_f32(slope));
}

int gk_gemm_packed_b_fused_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha, size_t m,
                                          const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                          const gk_packed_rhs *packed, gk_bf16 beta, gk_bf16 *c,
                                          ptrdiff_t rsc, ptrdiff_t csc, const gk_bf16 *bias,
                                          int32_t bias_dim, uint8_t has_bias, int32_t act,
                                          gk_bf16 slope, gk_par) {
    const FusedSpec fx{has_bias ? bias : nullptr, bias_dim, act, bf16_to_f32(slope)};
    return packed_b_unchecked(ws, InType::BF16, EpiKind::BF16, bf16_to_f32(alpha), m, a, rsa, csa,
                              packed, bf16_to_f32(beta), c, rsc, csc, &fx);
}

}  // extern "C"
