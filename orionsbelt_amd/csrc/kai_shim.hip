// kai_shim.hip -- the C ABI of libkai_gdn_hip.so.
//
// Two layers:
//  * kai_run_gdn_*_sve / _neon: the reference kai symbols with identical
//    prototypes (kleidiai_submission/kai/ukernels/gdn/*.h).  Synchronous;
//    each pointer may be host or device memory (hipPointerGetAttributes):
//    device pointers are used in place, host buffers are copied in/out.
//    The reference has no error channel (void returns; fatal conditions
//    print and exit(1), test_kai_gdn.c:38-42), so a HIP failure here prints
//    the failing call and exits(1).  seq==0 / channels==0 return before any
//    HIP call and write nothing (test_kai_gdn.c:520-637).
//  * kai_run_gdn_*_hip: device pointers, stream-ordered, return hipError_t
//    (include/kai_gdn_hip.h).
//
// Per-device state (created lazily under a mutex): an internal stream for
// the synchronous symbols, staging buffers, the look-back scan scratch and
// the prefill carry buffer.  Scan launches are serialised per device (host
// mutex; stream order, or a device synchronisation when the stream changes)
// because they share the tile counter and status arrays; every other kernel
// is free of shared state.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <new>
#include <vector>

#include "gdn_internal.h"
#include "../../include/gdn_sve.h"
#include "../../include/kai_gdn_hip.h"
#include "../../include/kai/ukernels/gdn/kai_gdn_causal_dwconv1d_f32_k4_sve.h"
#include "../../include/kai/ukernels/gdn/kai_gdn_cumdecay_f32_sve.h"
#include "../../include/kai/ukernels/gdn/kai_gdn_gated_scan_f32_sve.h"
#include "../../include/kai/ukernels/gdn/kai_gdn_gemv_f32_f32_f32_1x4_neon.h"
#include "../../include/gdn_delta_matmul.h"

namespace {

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    // grow to at least n bytes; the old contents are not kept
    hipError_t reserve(size_t n) {
        if (n <= cap) return hipSuccess;
        if (p) {
            hipError_t e = hipFree(p);
            if (e != hipSuccess) return e;
            p = nullptr;
            cap = 0;
        }
        size_t want = n < 4096 ? 4096 : n + n / 4;
        hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) return e;
        cap = want;
        return hipSuccess;
    }
};

struct DeviceCtx {
    std::mutex mu;        // serialises scan launches and buffer growth
    bool ready = false;
    hipStream_t stream = nullptr;
    // synchronous-path staging (one buffer per argument slot)
    DevBuf stage[6];
    // look-back scan scratch
    gdn::ScanScratch scan{};
    size_t scan_words = 0;
    unsigned long long counter_value = 0;
    uint32_t epoch = 0;
    // the last scan launch: its stream, and whether it may still be running
    hipStream_t scan_stream = nullptr;
    bool scan_pending = false;
    // GDN-2 gate products (g * b, w * x) feeding the gated scan
    DevBuf gdn2_tmp;
    // prefill carry buffer (segment transitions and start states)
    DevBuf chunk_ws;
    hipStream_t pf_stream = nullptr;  // stream of the last prefill
    bool pf_pending = false;
};

std::mutex g_ctx_mu;
std::vector<DeviceCtx *> g_ctx;

hipError_t get_ctx(DeviceCtx **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    DeviceCtx *c;
    {
        std::lock_guard<std::mutex> lk(g_ctx_mu);
        try {  // no C++ exception may cross the C ABI
            if ((int)g_ctx.size() <= dev) g_ctx.resize(dev + 1, nullptr);
        } catch (...) {
            return hipErrorOutOfMemory;
        }
        if (!g_ctx[dev]) g_ctx[dev] = new (std::nothrow) DeviceCtx();
        if (!g_ctx[dev]) return hipErrorOutOfMemory;
        c = g_ctx[dev];
    }
    std::lock_guard<std::mutex> lk(c->mu);
    if (!c->ready) {
        e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) return e;
        e = hipMalloc(&c->scan.counter, 256);
        if (e != hipSuccess) return e;
        e = hipMemset(c->scan.counter, 0, 256);
        if (e != hipSuccess) return e;
        c->scan.err = reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(c->scan.counter) + 64);
        e = hipDeviceGetAttribute(&c->scan.cu_count, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        c->ready = true;
    }
    *out = c;
    return hipSuccess;
}

// Grow the three scan status arrays to `words` entries each (zero-filled).
// Called with c->mu held.  Waits for the previous scan before freeing.
hipError_t scan_reserve(DeviceCtx *c, size_t words) {
    if (words <= c->scan_words) return hipSuccess;
    hipError_t e;
    if (c->scan_pending) {
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return e;
        c->scan_pending = false;
    }
    if (c->scan.incl) {
        (void)hipFree(c->scan.incl);
        c->scan.incl = c->scan.aggG = c->scan.aggX = nullptr;
        c->scan_words = 0;
    }
    size_t want = words < 65536 ? 65536 : words + words / 4;
    void *p = nullptr;
    e = hipMalloc(&p, 3 * want * sizeof(unsigned long long));
    if (e != hipSuccess) return e;
    e = hipMemset(p, 0, 3 * want * sizeof(unsigned long long));
    if (e != hipSuccess) return e;
    c->scan.incl = static_cast<unsigned long long *>(p);
    c->scan.aggG = c->scan.incl + want;
    c->scan.aggX = c->scan.aggG + want;
    c->scan_words = want;
    c->scan.words = want;
    c->epoch = 0;  // fresh arrays: restart tags
    return hipSuccess;
}

// A scan launch on `st`; called with c->mu held.
hipError_t run_scan_locked(DeviceCtx *c, int mode, int narrow, const float *g, const float *x, void *out,
                           void *state, size_t seq, size_t ch, hipStream_t st) {
    hipError_t e;
    const size_t nr = gdn::scan_row_tiles(seq, mode);
    e = scan_reserve(c, nr * ch);
    if (e != hipSuccess) return e;
    if (c->epoch == 0xFFFFFFFFu) {  // tag space exhausted: clear and restart
        if (c->scan_pending && (e = hipDeviceSynchronize()) != hipSuccess) return e;
        c->scan_pending = false;
        e = hipMemset(c->scan.incl, 0, 3 * c->scan_words * sizeof(unsigned long long));
        if (e != hipSuccess) return e;
        c->epoch = 0;
    }
    const uint32_t epoch = ++c->epoch;
    const unsigned long long base = c->counter_value;
    // Scans share the counter and status words, so a scan must not start
    // before the previous one ends.  On the same stream, stream order does
    // that at no cost (an event after every launch costs about 5 us here).
    // On another stream, the previous stream may no longer exist, so wait
    // for the device.
    if (c->scan_pending && st != c->scan_stream) {
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return e;
        c->scan_pending = false;
    }
    unsigned long long used = 0;
    e = gdn::launch_lookback_scan(mode, narrow, g, x, out, state, seq, ch, c->scan, base, epoch,
                                  &used, st);
    if (e != hipSuccess) return e;
    c->counter_value += used;
    c->scan_stream = st;
    c->scan_pending = true;
    return hipSuccess;
}

hipError_t run_scan(int mode, int narrow, const float *g, const float *x, void *out,
                    void *state, size_t seq, size_t ch, hipStream_t st) {
    if (seq == 0 || ch == 0) return hipSuccess;
    DeviceCtx *c;
    hipError_t e = get_ctx(&c);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(c->mu);
    return run_scan_locked(c, mode, narrow, g, x, out, state, seq, ch, st);
}

// GDN-2 scan: the gate products into the device's gdn2 buffers, then the
// gated scan over them.  The buffers are shared by every call on the device,
// so a call waits for a scan still running on another stream (it may be
// reading them), and growth waits for the device.
hipError_t run_gdn2(const float *g, const float *b, const float *w, const float *x, float *s, float *state,
                    size_t seq, size_t ch, hipStream_t st) {
    if (seq == 0 || ch == 0) return hipSuccess;
    DeviceCtx *c;
    hipError_t e = get_ctx(&c);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(c->mu);
    const size_t n = seq * ch;
    if (c->scan_pending && (st != c->scan_stream || 2 * n * sizeof(float) > c->gdn2_tmp.cap)) {
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return e;
        c->scan_pending = false;
    }
    e = c->gdn2_tmp.reserve(2 * n * sizeof(float));
    if (e != hipSuccess) return e;
    float *gp = static_cast<float *>(c->gdn2_tmp.p), *xp = gp + n;
    e = gdn::launch_gdn2_gates(g, b, w, x, gp, xp, n, st);
    if (e != hipSuccess) return e;
    return run_scan_locked(c, 1, gdn::kF32, gp, xp, s, state, seq, ch, st);
}

// ---- cumulative decay without allocation -----------------------------------
// The look-back scan's scratch for kai_run_gdn_cumdecay_f32_noalloc_hip lives
// in a file-scope device array of fixed size instead of hipMalloc'd memory:
// words [0, kNaHeader) hold the tile counter (word 0) and the error word
// (word 8), then three status arrays of kNaStatusWords words each.  Each GPU
// holds its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, never device memory: every host use goes through the
// per-device address from hipGetSymbolAddress (NaDev::ptr).
constexpr size_t kNaStatusWords = KAI_GDN_NOALLOC_SCAN_MAX_WORDS;
constexpr size_t kNaHeader = 64;
constexpr size_t kNaWords = kNaHeader + 3 * kNaStatusWords;
static __device__ __align__(256) unsigned long long scratch[kNaWords];

// Zero `n` 64-bit words (a kernel, not hipMemsetAsync: callers of the
// no-allocation entry point may capture it into a graph).
__global__ void na_zero_kernel(unsigned long long *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0ull;
}

struct NaDev {
    std::mutex mu;
    bool ready = false;
    unsigned long long *ptr = nullptr;   // device address of this GPU's `scratch`
    int cu_count = 0;
    uint32_t epoch = 0;                  // tag of the last launch's status words
    unsigned long long counter = 0;      // value of the tile counter after the last launch
};
constexpr int kNaMaxDevices = 64;
NaDev g_na[kNaMaxDevices];

// Per-device set-up, once, with the device current: the array's address and
// its contents cleared.  No allocation (hipGetSymbolAddress, a kernel launch
// and a device synchronisation).
hipError_t na_dev(NaDev **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kNaMaxDevices) return hipErrorInvalidDevice;
    NaDev *d = &g_na[dev];
    std::lock_guard<std::mutex> lk(d->mu);
    if (!d->ready) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        e = hipDeviceGetAttribute(&d->cu_count, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        na_zero_kernel<<<256, 256, 0, nullptr>>>(static_cast<unsigned long long *>(p), kNaWords);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return e;
        d->ptr = static_cast<unsigned long long *>(p);
        d->epoch = 0;
        d->counter = 0;
        d->ready = true;
    }
    *out = d;
    return hipSuccess;
}

// The device's no-allocation error word, or nullptr before its set-up.
uint32_t *na_err_word(int dev) {
    if (dev < 0 || dev >= kNaMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_na[dev].mu);
    return g_na[dev].ready ? reinterpret_cast<uint32_t *>(g_na[dev].ptr + 8) : nullptr;
}

// ---- synchronous (kai) path helpers ----------------------------------------

bool is_device_ptr(const void *p) {
    if (!p) return false;
    hipPointerAttribute_t a;
    hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

[[noreturn]] void fatal(const char *what, hipError_t e) {
    std::fprintf(stderr, "libkai_gdn_hip: %s failed: %s (%d)\n", what, hipGetErrorString(e), (int)e);
    std::exit(1);
}

void check(hipError_t e, const char *what) {
    if (e != hipSuccess) fatal(what, e);
}

// One argument of a synchronous call: a device view of `bytes` at `host`.
struct Arg {
    void *dev = nullptr;
    const void *src = nullptr;
    void *dst = nullptr;  // copy back on exit (outputs / in-out)
    size_t bytes = 0;
};

// in: copy to device before; out: copy back after.
Arg stage_arg(DeviceCtx *c, int slot, const void *p, size_t bytes, bool in, bool out) {
    Arg a;
    a.bytes = bytes;
    if (is_device_ptr(p)) {
        a.dev = const_cast<void *>(p);
        return a;
    }
    check(c->stage[slot].reserve(bytes), "hipMalloc (staging)");
    a.dev = c->stage[slot].p;
    if (in) check(hipMemcpyAsync(a.dev, p, bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync H2D");
    if (out) a.dst = const_cast<void *>(p);
    return a;
}

void finish(DeviceCtx *c, Arg *args, int n) {
    for (int i = 0; i < n; ++i)
        if (args[i].dst)
            check(hipMemcpyAsync(args[i].dst, args[i].dev, args[i].bytes, hipMemcpyDeviceToHost, c->stream),
                  "hipMemcpyAsync D2H");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

// After a synchronous call has drained the internal stream: a scan launched
// there has ended.  A look-back wait that gave up leaves the error word set
// and the output invalid; the synchronous symbols have no error channel, so
// that is fatal here (the reference's convention, test_kai_gdn.c:38-42).
void scan_settled(DeviceCtx *c) {
    std::lock_guard<std::mutex> lk(c->mu);
    if (c->scan_stream == c->stream) c->scan_pending = false;
    uint32_t err = 0;
    check(hipMemcpy(&err, c->scan.err, sizeof err, hipMemcpyDeviceToHost), "hipMemcpy (scan error word)");
    if (err) {
        (void)hipMemset(c->scan.err, 0, sizeof err);
        std::fprintf(stderr, "libkai_gdn_hip: a scan's look-back wait timed out (error word %u)\n", err);
        std::exit(1);
    }
}

DeviceCtx *sync_ctx() {
    DeviceCtx *c;
    check(get_ctx(&c), "HIP initialisation");
    return c;
}

// The synchronous symbols share the per-device staging buffers: one call at a
// time per process.
std::mutex g_sync_mu;

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

// ===========================================================================
// Library
// ===========================================================================

extern "C" int kai_gdn_hip_init(void) {
    DeviceCtx *c;
    hipError_t e = get_ctx(&c);
    if (e != hipSuccess) return (int)e;
    NaDev *d;
    return (int)na_dev(&d);
}

extern "C" const char *kai_gdn_hip_error_string(int code) {
    return hipGetErrorString((hipError_t)code);
}

extern "C" int kai_gdn_hip_check_device_error(void) {
    DeviceCtx *c;
    if (get_ctx(&c) != hipSuccess) return -1;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    uint32_t v = 0;
    if (hipMemcpy(&v, c->scan.err, sizeof v, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (v) (void)hipMemset(c->scan.err, 0, sizeof v);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    if (uint32_t *na = na_err_word(dev)) {  // the no-allocation scan's error word
        uint32_t w = 0;
        if (hipMemcpy(&w, na, sizeof w, hipMemcpyDeviceToHost) != hipSuccess) return -1;
        if (w) (void)hipMemset(na, 0, sizeof w);
        v |= w;
    }
    return (int)v;
}

extern "C" size_t kai_gdn_hip_prefill_workspace_bytes(int batch, int seq_len, int num_v_heads) {
    if (batch <= 0 || seq_len <= 0 || num_v_heads <= 0) return 0;
    return gdn::prefill_carry_bytes(batch, seq_len, num_v_heads);
}

extern "C" int kai_gdn_hip_prefill_windowed_heads(void) {
    DeviceCtx *c;
    if (get_ctx(&c) != hipSuccess) return -1;
    std::lock_guard<std::mutex> lk(c->mu);
    return gdn::prefill_windowed_heads();
}

extern "C" size_t kai_gdn_hip_device_bytes_held(void) {
    DeviceCtx *c;
    if (get_ctx(&c) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lk(c->mu);
    size_t n = 256 + c->chunk_ws.cap + c->gdn2_tmp.cap;  // 256: the scan counter and error word
    for (const DevBuf &s : c->stage) n += s.cap;
    return n + 3 * c->scan_words * sizeof(unsigned long long);
}

extern "C" size_t kai_gdn_hip_probe_sink_bytes(void) {
    DeviceCtx *c;
    if (get_ctx(&c) != hipSuccess) return 0;
    return gdn::probe_sink_words(c->scan.cu_count) * 4;
}

extern "C" int kai_gdn_hip_probe_stream(const void *src, void *dst, size_t bytes, int mode, void *sink,
                                        void *stream) {
    DeviceCtx *c;
    hipError_t e = get_ctx(&c);
    if (e != hipSuccess) return (int)e;
    if (!src || !sink || (mode == 0 && !dst) || (mode != 0 && mode != 1) || bytes % 16 != 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0 || (mode == 0 && reinterpret_cast<uintptr_t>(dst) % 16 != 0))
        return (int)hipErrorInvalidValue;
    return (int)gdn::launch_probe_stream(src, dst, bytes, mode, static_cast<uint32_t *>(sink), c->scan.cu_count,
                                         (hipStream_t)stream);
}

extern "C" int kai_gdn_hip_probe_mfma_bf16(int iters, int shape, void *sink, unsigned long long *flops,
                                           void *stream) {
    DeviceCtx *c;
    hipError_t e = get_ctx(&c);
    if (e != hipSuccess) return (int)e;
    if (iters < 1 || (shape != 0 && shape != 1) || !sink || !flops) return (int)hipErrorInvalidValue;
    return (int)gdn::launch_probe_mfma(static_cast<float *>(sink), iters, shape, c->scan.cu_count, flops,
                                       (hipStream_t)stream);
}

// ===========================================================================
// Device-pointer entry points
// ===========================================================================

extern "C" int kai_run_gdn_cumdecay_f32_hip(const float *a, float *decay, size_t seq,
                                            size_t channels, void *stream) {
    return (int)run_scan(0, gdn::kF32, a, nullptr, decay, nullptr, seq, channels,
                         (hipStream_t)stream);
}

extern "C" int kai_run_gdn_cumdecay_f16_hip(const float *a, uint16_t *decay, size_t seq,
                                            size_t channels, void *stream) {
    return (int)run_scan(0, gdn::kF16, a, nullptr, decay, nullptr, seq, channels,
                         (hipStream_t)stream);
}

extern "C" int kai_run_gdn_cumdecay_bf16_hip(const float *a, uint16_t *decay, size_t seq,
                                             size_t channels, void *stream) {
    return (int)run_scan(0, gdn::kBF16, a, nullptr, decay, nullptr, seq, channels,
                         (hipStream_t)stream);
}

extern "C" int kai_run_gdn_cumdecay_f32_noalloc_hip(const float *a, float *decay, size_t seq,
                                                    size_t channels, void *stream) {
    if (seq == 0 || channels == 0) return 0;
    if (!a || !decay) return (int)hipErrorInvalidValue;
    // beyond the fixed scratch: one status word per (row tile, channel)
    const size_t nr = gdn::scan_row_tiles(seq, 0);
    if (channels > kNaStatusWords || nr > kNaStatusWords / channels) return (int)hipErrorInvalidValue;
    NaDev *d;
    hipError_t e = na_dev(&d);
    if (e != hipSuccess) return (int)e;
    const hipStream_t st = (hipStream_t)stream;
    std::lock_guard<std::mutex> lk(d->mu);
    unsigned long long *hdr = d->ptr;
    unsigned long long *incl = hdr + kNaHeader;
    if (d->epoch == 0xFFFFFFFFu) {  // tag space exhausted: clear the status words, restart tags
        na_zero_kernel<<<1024, 256, 0, st>>>(incl, 3 * kNaStatusWords);
        if ((e = hipGetLastError()) != hipSuccess) return (int)e;
        d->epoch = 0;
    }
    gdn::ScanScratch s{};
    s.counter = hdr;
    s.err = reinterpret_cast<uint32_t *>(hdr + 8);
    s.incl = incl;
    s.aggG = incl + kNaStatusWords;
    s.aggX = incl + 2 * kNaStatusWords;
    s.words = kNaStatusWords;
    s.cu_count = d->cu_count;
    const uint32_t epoch = d->epoch + 1;
    unsigned long long used = 0;
    e = gdn::launch_lookback_scan(0, gdn::kF32, a, nullptr, decay, nullptr, seq, channels, s, d->counter,
                                  epoch, &used, st);
    if (e != hipSuccess) return (int)e;
    d->epoch = epoch;
    d->counter += used;
    return 0;
}

extern "C" int kai_run_gdn_gated_scan_f32_hip(const float *g, const float *x, float *s,
                                              float *state, size_t seq, size_t channels,
                                              void *stream) {
    return (int)run_scan(1, gdn::kF32, g, x, s, state, seq, channels, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_gated_scan_f16_hip(const float *g, const float *x, float *s,
                                              uint16_t *state, size_t seq, size_t channels,
                                              void *stream) {
    return (int)run_scan(1, gdn::kF16, g, x, s, state, seq, channels, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_gated_scan_bf16_hip(const float *g, const float *x, float *s,
                                               uint16_t *state, size_t seq, size_t channels,
                                               void *stream) {
    return (int)run_scan(1, gdn::kBF16, g, x, s, state, seq, channels, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_causal_dwconv1d_f32_k4_hip(const float *in, const float *w,
                                                      float *out, float *hist, size_t seq,
                                                      size_t channels, void *stream) {
    return (int)gdn::launch_conv_k4(in, w, out, hist, seq, channels, false, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip(const float *in, const float *w,
                                                           float *out, float *hist, size_t seq,
                                                           size_t channels, void *stream) {
    return (int)gdn::launch_conv_k4(in, w, out, hist, seq, channels, true, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_delta_rule_matmul_f32_hip(const float *A, const float *B, float *C, size_t M,
                                                     size_t K, size_t N, void *stream) {
    if (M == 0 || N == 0) return 0;
    if (!C || (K > 0 && (!A || !B))) return (int)hipErrorInvalidValue;
    return (int)gdn::launch_matmul(A, B, C, M, K, N, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_gemv_f32_f32_f32_hip(const float *a, const float *b, float *c,
                                                size_t k, size_t n, void *stream) {
    return (int)gdn::launch_gemv(a, b, c, k, n, (hipStream_t)stream);
}

static int check_decode_args(const void *S, const float *q, const float *k, const float *v,
                             const float *g, const float *beta, const float *o, int B, int Hv,
                             int Hk, int dk, int dv, size_t s_align) {
    if (B < 0 || Hv < 0 || Hk <= 0 || (Hv > 0 && Hv % Hk != 0)) return (int)hipErrorInvalidValue;
    const bool dims_ok = (dk == 32 || dk == 64 || dk == 128) && (dv == 32 || dv == 64 || dv == 128);
    if (!dims_ok) return (int)hipErrorInvalidValue;
    if (B == 0 || Hv == 0) return 0;
    if (!S || !q || !k || !v || !g || !beta || !o) return (int)hipErrorInvalidValue;
    if (!aligned(S, s_align) || !aligned(v, 16) || !aligned(o, 16)) return (int)hipErrorInvalidValue;
    return 0;
}

extern "C" int kai_run_gdn_delta_rule_decode_f32_hip(float *S, const float *q, const float *k,
                                                     const float *v, const float *g,
                                                     const float *beta, float *o, int batch,
                                                     int num_v_heads, int num_k_heads,
                                                     int head_k_dim, int head_v_dim,
                                                     float q_scale, void *stream) {
    int rc = check_decode_args(S, q, k, v, g, beta, o, batch, num_v_heads, num_k_heads,
                               head_k_dim, head_v_dim, 16);
    if (rc) return rc;
    return (int)gdn::launch_delta_decode(gdn::kF32, S, q, k, v, g, beta, o, batch, num_v_heads,
                                         num_k_heads, head_k_dim, head_v_dim, q_scale,
                                         (hipStream_t)stream);
}

extern "C" int kai_run_gdn_delta_rule_decode_f16state_hip(uint16_t *S, const float *q,
                                                          const float *k, const float *v,
                                                          const float *g, const float *beta,
                                                          float *o, int batch, int num_v_heads,
                                                          int num_k_heads, int head_k_dim,
                                                          int head_v_dim, float q_scale,
                                                          void *stream) {
    int rc = check_decode_args(S, q, k, v, g, beta, o, batch, num_v_heads, num_k_heads,
                               head_k_dim, head_v_dim, 8);
    if (rc) return rc;
    return (int)gdn::launch_delta_decode(gdn::kF16, S, q, k, v, g, beta, o, batch, num_v_heads,
                                         num_k_heads, head_k_dim, head_v_dim, q_scale,
                                         (hipStream_t)stream);
}

static int run_chunk(int narrow, const uint16_t *q, const uint16_t *k, const uint16_t *v,
                     const float *g, const float *beta, uint16_t *o, void *S, int B, int T,
                     int Hv, int Hk, float q_scale, hipStream_t st) {
    if (B < 0 || T < 0 || Hv < 0 || Hk <= 0 || (Hv > 0 && Hv % Hk != 0))
        return (int)hipErrorInvalidValue;
    if (B == 0 || T == 0 || Hv == 0) return 0;
    if (!q || !k || !v || !g || !beta || !o || !S) return (int)hipErrorInvalidValue;
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16)) return (int)hipErrorInvalidValue;
    DeviceCtx *c;
    hipError_t e = get_ctx(&c);
    if (e != hipSuccess) return (int)e;
    std::lock_guard<std::mutex> lk(c->mu);
    const size_t need = gdn::prefill_carry_bytes(B, T, Hv);
    if (need > c->chunk_ws.cap) {
        // a previous prefill may still be using the old carry buffer
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return (int)e;
        c->pf_pending = false;
        e = c->chunk_ws.reserve(need);
        if (e != hipSuccess) return (int)e;
    }
    // Calls share the carry buffer, so a call must not start before the
    // previous one ends: stream order does that on the same stream; on
    // another stream (the previous one may no longer exist) wait for the
    // device.
    if (c->pf_pending && st != c->pf_stream) {
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return (int)e;
        c->pf_pending = false;
    }
    e = gdn::launch_prefill_seq(narrow, q, k, v, g, beta, o, S, B, T, Hv, Hk, q_scale,
                                c->chunk_ws.p, st);
    if (e != hipSuccess) return (int)e;
    c->pf_stream = st;
    c->pf_pending = true;
    return 0;
}

extern "C" int kai_run_gdn_chunk_delta_rule_bf16_f32_hip(const uint16_t *q, const uint16_t *k,
                                                         const uint16_t *v, const float *g,
                                                         const float *beta, uint16_t *o,
                                                         float *S, int batch, int seq_len,
                                                         int num_v_heads, int num_k_heads,
                                                         float q_scale, void *stream) {
    return run_chunk(gdn::kF32, q, k, v, g, beta, o, S, batch, seq_len, num_v_heads, num_k_heads,
                     q_scale, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_chunk_delta_rule_bf16_f16state_hip(
    const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *g, const float *beta,
    uint16_t *o, uint16_t *S, int batch, int seq_len, int num_v_heads, int num_k_heads,
    float q_scale, void *stream) {
    return run_chunk(gdn::kF16, q, k, v, g, beta, o, S, batch, seq_len, num_v_heads, num_k_heads,
                     q_scale, (hipStream_t)stream);
}

// ---- layer glue: gating prologue and gated RMSNorm ------------------------

static int check_prologue_args(const float *x, const float *a, const float *b, const float *A_log,
                               const float *dt_bias, const void *q, const void *k, const void *v,
                               const float *g, const float *beta, size_t rows, int Hk, int Hv,
                               size_t out_align) {  // 16-byte accesses to every array
    if (Hk <= 0 || Hv <= 0 || Hv % Hk != 0) return (int)hipErrorInvalidValue;
    if (rows == 0) return 0;
    if (rows > 0x7FFFFFFFu) return (int)hipErrorInvalidValue;
    if (!x || !a || !b || !A_log || !dt_bias || !q || !k || !v || !g || !beta)
        return (int)hipErrorInvalidValue;
    if (!aligned(x, 16) || !aligned(q, out_align) || !aligned(k, out_align) || !aligned(v, out_align))
        return (int)hipErrorInvalidValue;
    return 0;
}

extern "C" int kai_run_gdn_gating_prologue_bf16_hip(const float *x, const float *a, const float *b,
                                                    const float *A_log, const float *dt_bias,
                                                    uint16_t *q, uint16_t *k, uint16_t *v, float *g,
                                                    float *beta, size_t rows, int num_k_heads,
                                                    int num_v_heads, void *stream) {
    int rc = check_prologue_args(x, a, b, A_log, dt_bias, q, k, v, g, beta, rows, num_k_heads,
                                 num_v_heads, 16);
    if (rc || rows == 0) return rc;
    return (int)gdn::launch_gating_prologue(true, x, a, b, A_log, dt_bias, q, k, v, g, beta, rows,
                                            num_k_heads, num_v_heads, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_gating_prologue_f32_hip(const float *x, const float *a, const float *b,
                                                   const float *A_log, const float *dt_bias,
                                                   float *q, float *k, float *v, float *g,
                                                   float *beta, size_t rows, int num_k_heads,
                                                   int num_v_heads, void *stream) {
    int rc = check_prologue_args(x, a, b, A_log, dt_bias, q, k, v, g, beta, rows, num_k_heads,
                                 num_v_heads, 16);
    if (rc || rows == 0) return rc;
    return (int)gdn::launch_gating_prologue(false, x, a, b, A_log, dt_bias, q, k, v, g, beta, rows,
                                            num_k_heads, num_v_heads, (hipStream_t)stream);
}

static int check_rmsnorm_args(const void *o, const void *z, const void *w, const void *y,
                              size_t rows, float eps, size_t align) {
    if (!(eps >= 0.0f)) return (int)hipErrorInvalidValue;  // also rejects NaN
    if (rows == 0) return 0;
    if (!o || !z || !w || !y) return (int)hipErrorInvalidValue;
    if (!aligned(o, align) || !aligned(z, align) || !aligned(w, align) || !aligned(y, align))
        return (int)hipErrorInvalidValue;
    return 0;
}

extern "C" int kai_run_gdn_gated_rmsnorm_bf16_hip(const uint16_t *o, const uint16_t *z,
                                                  const uint16_t *w, uint16_t *y, size_t rows,
                                                  float eps, void *stream) {
    int rc = check_rmsnorm_args(o, z, w, y, rows, eps, 16);
    if (rc || rows == 0) return rc;
    return (int)gdn::launch_gated_rmsnorm(true, o, z, w, y, rows, eps, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_gated_rmsnorm_f32_hip(const float *o, const float *z, const float *w,
                                                 float *y, size_t rows, float eps, void *stream) {
    int rc = check_rmsnorm_args(o, z, w, y, rows, eps, 16);
    if (rc || rows == 0) return rc;
    return (int)gdn::launch_gated_rmsnorm(false, o, z, w, y, rows, eps, (hipStream_t)stream);
}

// ---- state hand-off formats and the decode-step conv -----------------------

static int check_conv_state_args(int B, size_t C, const void *state, std::initializer_list<const void *> others) {
    if (B < 0 || B > 65535) return (int)hipErrorInvalidValue;
    if (B == 0 || C == 0) return 0;
    if (C > ((size_t)1 << 40)) return (int)hipErrorInvalidValue;
    if (!state || !aligned(state, 16)) return (int)hipErrorInvalidValue;
    for (const void *p : others)
        if (!p) return (int)hipErrorInvalidValue;
    return 0;
}

extern "C" int kai_run_gdn_causal_conv1d_update_f32_hip(const float *x, float *conv_state,
                                                        const float *w, float *out, int batch,
                                                        int seq_len, size_t channels, int silu,
                                                        void *stream) {
    if (seq_len < 0) return (int)hipErrorInvalidValue;
    int rc = check_conv_state_args(batch, channels, conv_state, {x, w, out});
    if (rc || batch == 0 || channels == 0 || seq_len == 0) return rc;
    if (!aligned(w, 16)) return (int)hipErrorInvalidValue;
    return (int)gdn::launch_conv_update(x, conv_state, w, out, batch, seq_len, channels, silu != 0,
                                        (hipStream_t)stream);
}

extern "C" int kai_run_gdn_conv_state_from_inputs_f32_hip(const float *x, float *conv_state,
                                                          int batch, size_t seq_len,
                                                          size_t channels, void *stream) {
    int rc = check_conv_state_args(batch, channels, conv_state, {seq_len ? x : conv_state});
    if (rc || batch == 0 || channels == 0) return rc;
    return (int)gdn::launch_conv_state_from_inputs(x, conv_state, batch, seq_len, channels,
                                                   (hipStream_t)stream);
}

extern "C" int kai_run_gdn_conv_state_to_hist_f32_hip(const float *conv_state, float *hist,
                                                      int batch, size_t channels, void *stream) {
    int rc = check_conv_state_args(batch, channels, conv_state, {hist});
    if (rc || batch == 0 || channels == 0) return rc;
    return (int)gdn::launch_conv_hist_state(true, hist, const_cast<float *>(conv_state), batch,
                                            channels, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_conv_hist_to_state_f32_hip(const float *hist, float *conv_state,
                                                      int batch, size_t channels, void *stream) {
    int rc = check_conv_state_args(batch, channels, conv_state, {hist});
    if (rc || batch == 0 || channels == 0) return rc;
    return (int)gdn::launch_conv_hist_state(false, const_cast<float *>(hist), conv_state, batch,
                                            channels, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_state_convert_hip(const void *src, int src_format, void *dst,
                                             int dst_format, size_t count, void *stream) {
    auto ok = [](int f) { return f == gdn::kF32 || f == gdn::kF16 || f == gdn::kBF16; };
    if (!ok(src_format) || !ok(dst_format)) return (int)hipErrorInvalidValue;
    if (count == 0) return 0;
    if (!src || !dst) return (int)hipErrorInvalidValue;
    const size_t sb = count * (src_format == gdn::kF32 ? 4 : 2);
    const size_t db = count * (dst_format == gdn::kF32 ? 4 : 2);
    const uintptr_t s0 = (uintptr_t)src, d0 = (uintptr_t)dst;
    const bool same = s0 == d0 && src_format == dst_format;
    if (!same && s0 < d0 + db && d0 < s0 + sb) return (int)hipErrorInvalidValue;  // overlap
    return (int)gdn::launch_convert(src, src_format, dst, dst_format, count, (hipStream_t)stream);
}

// ---- hybrid decode loop: int8 weight-only matmul ---------------------------

extern "C" size_t kai_gdn_w8a16_gemm_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || N % 16 || K % 256) return 0;
    return gdn::w8_workspace_bytes(M, N, K);
}

extern "C" int kai_run_gdn_w8a16_gemm_hip(const uint16_t *x, const int8_t *Wq, const float *scale,
                                          float *y, int M, int N, int K, void *workspace,
                                          size_t workspace_bytes, void *stream) {
    if (M < 0 || M > 16 || N < 0 || K <= 0 || N % 16 || K % 256) return (int)hipErrorInvalidValue;
    if (M == 0 || N == 0) return 0;
    if (!x || !Wq || !scale || !y) return (int)hipErrorInvalidValue;
    if (!aligned(x, 16) || !aligned(Wq, 16) || !aligned(scale, 16) || !aligned(y, 16))
        return (int)hipErrorInvalidValue;
    const size_t need = gdn::w8_workspace_bytes(M, N, K);
    if (need && (!workspace || workspace_bytes < need || !aligned(workspace, 16)))
        return (int)hipErrorInvalidValue;
    return (int)gdn::launch_w8_gemm(x, Wq, scale, y, M, N, K, static_cast<float *>(workspace),
                                    (hipStream_t)stream);
}

extern "C" int kai_run_gdn_w8_tile_hip(const int8_t *Wq, int8_t *Wt, int N, int K, void *stream) {
    if (N < 0 || K <= 0 || N % 64 || K % 256) return (int)hipErrorInvalidValue;
    if (N == 0) return 0;
    if (!Wq || !Wt || Wq == Wt || !aligned(Wq, 16) || !aligned(Wt, 16)) return (int)hipErrorInvalidValue;
    return (int)gdn::launch_w8f_tile(Wq, Wt, N, K, (hipStream_t)stream);
}

// workspace: the split partials (floats), then N / 64 counters
static size_t w8f_ws_bytes(int M, int N, int K) {
    const size_t part = gdn::w8f_workspace_floats(M, N, K);
    return part ? (part * sizeof(float) + (size_t)(N / 64) * sizeof(uint32_t) + 255) / 256 * 256 : 0;
}

extern "C" size_t kai_gdn_w8a16_gemm_tiled_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || M > 16 || N <= 0 || K <= 0 || N % 64 || K % 256) return 0;
    return w8f_ws_bytes(M, N, K);
}

extern "C" int kai_run_gdn_w8a16_gemm_tiled_hip(const uint16_t *x, const int8_t *Wt, const float *scale, float *y,
                                                int M, int N, int K, void *workspace, size_t workspace_bytes,
                                                void *stream) {
    if (M < 0 || N < 0 || K <= 0 || N % 64 || K % 256) return (int)hipErrorInvalidValue;
    if (M == 0 || N == 0) return 0;
    if (!x || !Wt || !scale || !y) return (int)hipErrorInvalidValue;
    if (!aligned(x, 16) || !aligned(Wt, 16) || !aligned(scale, 16) || !aligned(y, 16))
        return (int)hipErrorInvalidValue;
    if (M > 16) {  // the prefill's many-row GEMM (no workspace)
        gdn::W8Out o{};
        o.seg[0] = gdn::W8Seg{y, N, N};
        o.nseg = 1;
        o.mode = gdn::kW8Segments;
        return (int)gdn::launch_w8p(x, K, Wt, scale, M, N, K, o, (hipStream_t)stream);
    }
    const size_t need = w8f_ws_bytes(M, N, K);
    if (need && (!workspace || workspace_bytes < need || !aligned(workspace, 256))) return (int)hipErrorInvalidValue;
    float *part = static_cast<float *>(workspace);
    uint32_t *cnt = need ? reinterpret_cast<uint32_t *>(part + gdn::w8f_workspace_floats(M, N, K)) : nullptr;
    gdn::W8Out o{};
    o.seg[0] = gdn::W8Seg{y, N, N};
    o.nseg = 1;
    o.mode = gdn::kW8Segments;
    return (int)gdn::launch_w8f(x, Wt, scale, M, N, K, o, part, cnt, (hipStream_t)stream);
}

extern "C" int kai_run_gdn_w8_quantize_hip(const float *W, int8_t *Wq, float *scale, int N, int K,
                                           void *stream) {
    if (N < 0 || K < 0) return (int)hipErrorInvalidValue;
    if (N == 0 || K == 0) return 0;
    if (!W || !Wq || !scale) return (int)hipErrorInvalidValue;
    return (int)gdn::launch_w8_quantize(W, Wq, scale, N, K, (hipStream_t)stream);
}

extern "C" size_t kai_gdn_attn_decode_workspace_bytes(int batch, int num_q_heads, int length) {
    if (batch <= 0 || num_q_heads <= 0 || length <= 0) return 0;
    return gdn::attn_workspace_bytes(batch, num_q_heads, length);
}

extern "C" int kai_run_gdn_attn_decode_f16kv_hip(const uint16_t *q, const uint16_t *k_cache,
                                                 const uint16_t *v_cache, float *out, int batch,
                                                 int num_q_heads, int num_kv_heads, int max_len,
                                                 int length, float scaling, void *workspace,
                                                 size_t workspace_bytes, void *stream) {
    if (batch < 0 || batch > 65535 || num_kv_heads <= 0 || num_q_heads <= 0 ||
        num_q_heads % num_kv_heads || num_q_heads / num_kv_heads > 4 || num_kv_heads > 65535)
        return (int)hipErrorInvalidValue;
    if (length <= 0 || length > max_len) return (int)hipErrorInvalidValue;
    if (batch == 0) return 0;
    if (!q || !k_cache || !v_cache || !out || !workspace) return (int)hipErrorInvalidValue;
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(out, 16) ||
        !aligned(workspace, 16))
        return (int)hipErrorInvalidValue;
    if (workspace_bytes < gdn::attn_workspace_bytes(batch, num_q_heads, length))
        return (int)hipErrorInvalidValue;
    return (int)gdn::launch_attn_decode(q, k_cache, v_cache, out, batch, num_q_heads, num_kv_heads,
                                        max_len, length, scaling, static_cast<float *>(workspace),
                                        (hipStream_t)stream);
}

// ===========================================================================
// Reference kai symbols (synchronous, host or device pointers)
// ===========================================================================

extern "C" void kai_run_gdn_cumdecay_f32_sve(const float *a, float *decay, size_t seq,
                                             size_t channels) {
    if (seq == 0 || channels == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    const size_t n = seq * channels * sizeof(float);
    Arg args[2] = {stage_arg(c, 0, a, n, true, false), stage_arg(c, 1, decay, n, false, true)};
    check(run_scan(0, gdn::kF32, (const float *)args[0].dev, nullptr, args[1].dev, nullptr, seq,
                   channels, c->stream),
          "cumdecay launch");
    finish(c, args, 2);
    scan_settled(c);
}

extern "C" void kai_run_gdn_gated_scan_f32_sve(const float *g, const float *x, float *s,
                                               float *state, size_t seq, size_t channels) {
    if (seq == 0 || channels == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    const size_t n = seq * channels * sizeof(float);
    Arg args[4] = {stage_arg(c, 0, g, n, true, false), stage_arg(c, 1, x, n, true, false),
                   stage_arg(c, 2, s, n, false, true),
                   stage_arg(c, 3, state, channels * sizeof(float), true, true)};
    check(run_scan(1, gdn::kF32, (const float *)args[0].dev, (const float *)args[1].dev,
                   args[2].dev, args[3].dev, seq, channels, c->stream),
          "gated_scan launch");
    finish(c, args, 4);
    scan_settled(c);
}

extern "C" void kai_run_gdn_causal_dwconv1d_f32_k4_sve(const float *in, const float *w,
                                                       float *out, float *hist, size_t seq,
                                                       size_t channels) {
    if (seq == 0 || channels == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    const size_t n = seq * channels * sizeof(float);
    Arg args[4] = {stage_arg(c, 0, in, n, true, false),
                   stage_arg(c, 1, w, 4 * channels * sizeof(float), true, false),
                   stage_arg(c, 2, out, n, false, true),
                   stage_arg(c, 3, hist, 3 * channels * sizeof(float), true, true)};
    check(gdn::launch_conv_k4((const float *)args[0].dev, (const float *)args[1].dev,
                              (float *)args[2].dev, (float *)args[3].dev, seq, channels, false,
                              c->stream),
          "dwconv1d launch");
    finish(c, args, 4);
}

extern "C" void kai_run_gdn_gemv_f32_f32_f32_1x4_neon(const float *a, const float *b, float *c_,
                                                      size_t k, size_t n) {
    if (n == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    Arg args[3] = {stage_arg(c, 0, a, (k ? k : 1) * sizeof(float), k > 0, false),
                   stage_arg(c, 1, b, (k ? k * n : 1) * sizeof(float), k > 0, false),
                   stage_arg(c, 2, c_, n * sizeof(float), false, true)};
    check(gdn::launch_gemv((const float *)args[0].dev, (const float *)args[1].dev,
                           (float *)args[2].dev, k, n, c->stream),
          "gemv launch");
    finish(c, args, 3);
}

// gdn_delta_rule_matmul (gdn_delta_matmul.h:15-16): the same staging as the
// kai symbols.
extern "C" void gdn_delta_rule_matmul(const float *A, const float *B, float *C_, size_t M, size_t K, size_t N) {
    if (M == 0 || N == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    Arg args[3] = {stage_arg(c, 0, A, (K ? M * K : 1) * sizeof(float), K > 0, false),
                   stage_arg(c, 1, B, (K ? K * N : 1) * sizeof(float), K > 0, false),
                   stage_arg(c, 2, C_, M * N * sizeof(float), false, true)};
    check(gdn::launch_matmul((const float *)args[0].dev, (const float *)args[1].dev, (float *)args[2].dev, M, K, N,
                             c->stream),
          "delta_rule_matmul launch");
    finish(c, args, 3);
}

// ===========================================================================
// The reference's gdn_* ABI (include/gdn_sve.h): synchronous, host or device
// pointers, like the kai symbols above.
// ===========================================================================

extern "C" void gdn_cumdecay_f32(const float *a, float *decay, size_t seq, size_t channels) {
    kai_run_gdn_cumdecay_f32_sve(a, decay, seq, channels);
}

extern "C" void gdn_gated_scan_f32(const float *g, const float *x, float *s, float *state, size_t seq,
                                   size_t channels) {
    kai_run_gdn_gated_scan_f32_sve(g, x, s, state, seq, channels);
}

extern "C" void gdn_causal_dwconv1d_f32(const float *in, const float *w, float *out, float *hist, size_t seq,
                                        size_t channels) {
    kai_run_gdn_causal_dwconv1d_f32_k4_sve(in, w, out, hist, seq, channels);
}

namespace {
void sync_narrow_decay(int narrow, const float *a, void *decay, size_t seq, size_t channels) {
    if (seq == 0 || channels == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    const size_t n = seq * channels;
    Arg args[2] = {stage_arg(c, 0, a, n * sizeof(float), true, false),
                   stage_arg(c, 1, decay, n * sizeof(uint16_t), false, true)};
    check(run_scan(0, narrow, (const float *)args[0].dev, nullptr, args[1].dev, nullptr, seq, channels, c->stream),
          "cumdecay launch");
    finish(c, args, 2);
    scan_settled(c);
}

void sync_narrow_scan(int narrow, const float *g, const float *x, float *s, void *state, size_t seq,
                      size_t channels) {
    if (seq == 0 || channels == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    const size_t n = seq * channels * sizeof(float);
    Arg args[4] = {stage_arg(c, 0, g, n, true, false), stage_arg(c, 1, x, n, true, false),
                   stage_arg(c, 2, s, n, false, true),
                   stage_arg(c, 3, state, channels * sizeof(uint16_t), true, true)};
    check(run_scan(1, narrow, (const float *)args[0].dev, (const float *)args[1].dev, args[2].dev, args[3].dev,
                   seq, channels, c->stream),
          "gated_scan launch");
    finish(c, args, 4);
    scan_settled(c);
}
}  // namespace

extern "C" void gdn_cumdecay_f16(const float *a, GDN_SVE_F16 *decay, size_t seq, size_t channels) {
    sync_narrow_decay(gdn::kF16, a, decay, seq, channels);
}
extern "C" void gdn_cumdecay_bf16(const float *a, uint16_t *decay, size_t seq, size_t channels) {
    sync_narrow_decay(gdn::kBF16, a, decay, seq, channels);
}
extern "C" void gdn_gated_scan_f16(const float *g, const float *x, float *s, GDN_SVE_F16 *state, size_t seq,
                                   size_t channels) {
    sync_narrow_scan(gdn::kF16, g, x, s, state, seq, channels);
}
extern "C" void gdn_gated_scan_bf16(const float *g, const float *x, float *s, uint16_t *state, size_t seq,
                                    size_t channels) {
    sync_narrow_scan(gdn::kBF16, g, x, s, state, seq, channels);
}

extern "C" void gdn2_gated_scan_f32(const float *g, const float *b_gate, const float *w_gate, const float *x,
                                    float *s, float *state, size_t seq, size_t channels) {
    if (seq == 0 || channels == 0) return;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    DeviceCtx *c = sync_ctx();
    const size_t n = seq * channels * sizeof(float);
    Arg args[6] = {stage_arg(c, 0, g, n, true, false),      stage_arg(c, 1, b_gate, n, true, false),
                   stage_arg(c, 2, w_gate, n, true, false), stage_arg(c, 3, x, n, true, false),
                   stage_arg(c, 4, s, n, false, true),
                   stage_arg(c, 5, state, channels * sizeof(float), true, true)};
    check(run_gdn2((const float *)args[0].dev, (const float *)args[1].dev, (const float *)args[2].dev,
                   (const float *)args[3].dev, (float *)args[4].dev, (float *)args[5].dev, seq, channels, c->stream),
          "gdn2 gated_scan launch");
    finish(c, args, 6);
    scan_settled(c);
}

extern "C" int kai_run_gdn2_gated_scan_f32_hip(const float *g, const float *b_gate, const float *w_gate,
                                               const float *x, float *s, float *state, size_t seq, size_t channels,
                                               void *stream) {
    if (seq == 0 || channels == 0) return 0;
    if (!g || !b_gate || !w_gate || !x || !s || !state) return (int)hipErrorInvalidValue;
    return (int)run_gdn2(g, b_gate, w_gate, x, s, state, seq, channels, (hipStream_t)stream);
}
