// C ABI of the gfx950 quantized-matmul backend (include/fuel_rocm.h): device
// handles, quantized storages (the DynQuantizedStorage / QuantizedDeviceKernels
// mirror) and the KernelRef-shaped qmatmul.  Host code only.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/fuel_rocm.h"
#include "common.hpp"
#include "gguf.hpp"
#include "kernels.hpp"

using namespace frq;

// Scratch of frq_qmatmul_noalloc: quantized activation rows and split-K
// partial sums, in a device array of fixed size rather than the handle's
// hipMalloc'd workspace.  Every GPU the library runs on holds its own copy
// until the process ends.  In host code the array's name is only a stand-in:
// its device address (per GPU) comes from hipGetSymbolAddress at
// frq_device_open and is what kernels are given.
constexpr size_t FRQ_NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[FRQ_NOALLOC_SCRATCH_BYTES];

struct frq_device {
    int ordinal = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int num_cus = 0;
    void* ws = nullptr;  // activation workspace (quantized rows)
    size_t ws_bytes = 0;
    void* scratch = nullptr;  // this device's copy of the allocation-free entry point's scratch array
    // references: the open handle plus one per live storage; the struct is
    // deleted when the last one is dropped (a storage may outlive close)
    std::atomic<int> refs{1};
    // held by every entry point that enqueues work on the device or touches
    // its stream or workspace: calls from several threads (on the handle or
    // on storages of the device) take turns on the host, and their work runs
    // in call order on the one stream, so a workspace grown by one call is
    // never freed under another's kernels (hipFree waits for them)
    std::recursive_mutex mu;
};

struct frq_gguf {
    std::unique_ptr<frq::gguf::File> f;
};

struct frq_qstorage {
    frq_device* dev = nullptr;
    int dtype = 0;
    size_t nbytes = 0;
    uint8_t* d_ptr = nullptr;
};

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                   \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return fail(FRQ_INTERNAL, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                        __LINE__);                                                      \
    } while (0)

size_t type_size(int t) {
    switch (t) {
        case GGML_Q8_0: return Q8_0_BYTES;
        case GGML_Q4K: return Q4K_BYTES;
        case GGML_Q6K: return Q6K_BYTES;
        case GGML_Q8K: return Q8K_BYTES;
        default: return 0;
    }
}

size_t block_elems(int t) {
    switch (t) {
        case GGML_Q8_0: return QK8_0;
        case GGML_Q4K:
        case GGML_Q6K:
        case GGML_Q8K: return QK_K;
        default: return 0;
    }
}

bool is_weight_type(int t) { return t == GGML_Q8_0 || t == GGML_Q4K || t == GGML_Q6K; }

// Activation dtype a weight type is dotted against (GgmlType::VecDotType).
int vec_dot_type(int t) { return t == GGML_Q8_0 ? GGML_Q8_0 : GGML_Q8K; }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Activation rows per call: one row takes the fused quantize + mat-vec; up to
// MMQ_MIN_ROWS - 1 rows the skinny MFMA kernel (one weight pass per 32-row
// group); from MMQ_MIN_ROWS rows the tiled int8-MFMA GEMM -- and from
// MMQ_WIDE_MIN_ROWS rows already when the matrix has at least MMQ_WIDE_N
// columns: the skinny kernel's 16-column workgroups each read every quantized
// row, which costs more than the tiles' partly empty rows once there are many
// columns (4096x32000: M = 16 36.3 -> 31.1 us, M = 32 56.4 -> 33.6 us;
// 4096x11008 M = 32 28.3 -> 21.3 us; at N = 4096 the skinny kernel stays
// faster, 12.7 against 15.0 us at M = 32).  Q4_K at a 16-byte aligned base
// (the wide-tile kernel) goes further: rows of at least MMQ_LONG_K elements
// from MMQ_LONG_MIN_ROWS rows (a K split: 11008x4096 M = 24 17.1 -> 15.5 us,
// M = 32 19.9 -> 15.6; at 16 rows the skinny kernel stays faster, 12.0
// against 14.5 us), and shorter rows of >= MMQ_WIDE_N columns from
// MMQ_FEW_MIN_ROWS rows (16-row tiles: 4096x11008 M = 8 15.7 -> 13.4 us,
// 4096x32000 M = 8 29.3 -> 19.8, quantize launch included) -- from
// MMQ_FEW_MIN_ROWS_XL rows with >= MMQ_XL_N columns, where they also beat
// the 4-row mat-vec (4096x32000 M = 4 23.8 -> 20.1 us; at 2 rows the
// mat-vec stays, 16.8 against about 18.5).  Q6_K takes its wide-tile kernel
// from MMQ_FEW_MIN_ROWS rows on matrices of >= MMQ_Q6K_WIDE_N columns and
// rows shorter than MMQ_LONG_K (4096x32000 M = 8 40.7 -> 32.7 us; with
// fewer columns its 16 x 64 tiles leave the chip short and the skinny kernel
// stays), and its 32-row plane tiles with a K split on rows of >= MMQ_LONG_K
// elements from MMQ_LONG_MIN_ROWS rows (11008x4096 M = 32 26.4 -> 22.0 us
// against the skinny kernel, quantize launch excluded; 21.2 against 19.7 at
// 16 rows).
constexpr size_t MMQ_MIN_ROWS = 33;
constexpr size_t MMQ_WIDE_MIN_ROWS = 16;
constexpr size_t MMQ_WIDE_N = 8192;
constexpr size_t MMQ_LONG_MIN_ROWS = 24;
constexpr size_t MMQ_LONG_K = 8192;
constexpr size_t MMQ_FEW_MIN_ROWS = 5;
constexpr size_t MMQ_FEW_MIN_ROWS_XL = 3;
constexpr size_t MMQ_XL_N = 16384;
constexpr size_t MMQ_Q6K_WIDE_N = 24576;
bool tiled_rows(int t, const void* w, size_t rows, size_t n, size_t k) {
    if (rows >= MMQ_MIN_ROWS || (rows >= MMQ_WIDE_MIN_ROWS && n >= MMQ_WIDE_N)) return true;
    if (t == GGML_Q6K)
        return k < MMQ_LONG_K ? rows >= MMQ_FEW_MIN_ROWS && n >= MMQ_Q6K_WIDE_N : rows >= MMQ_LONG_MIN_ROWS;
    if (t != GGML_Q4K || ((uintptr_t)w & 15u) != 0) return false;
    if (k >= MMQ_LONG_K) return rows >= MMQ_LONG_MIN_ROWS;
    return n >= MMQ_WIDE_N && (rows >= MMQ_FEW_MIN_ROWS || (rows >= MMQ_FEW_MIN_ROWS_XL && n >= MMQ_XL_N));
}

// Byte size of the quantized-activation workspace for rows x k.
size_t act_bytes(int vt, size_t rows, size_t k) {
    const size_t kb = k / block_elems(vt);
    size_t b = align256(rows * k);                       // qs
    b += align256(rows * kb * sizeof(float));            // d
    if (vt == GGML_Q8K) b += 2 * align256(rows * kb * 16 * sizeof(int16_t));  // bsums, bsh
    return b;
}

ActView act_view(void* base, int vt, size_t rows, size_t k) {
    const size_t kb = k / block_elems(vt);
    uint8_t* p = static_cast<uint8_t*>(base);
    ActView v;
    v.qs = reinterpret_cast<int8_t*>(p);
    p += align256(rows * k);
    v.d = reinterpret_cast<float*>(p);
    p += align256(rows * kb * sizeof(float));
    v.bsums = vt == GGML_Q8K ? reinterpret_cast<int16_t*>(p) : nullptr;
    v.bsh = vt == GGML_Q8K ? reinterpret_cast<uint16_t*>(p + align256(rows * kb * 16 * sizeof(int16_t))) : nullptr;
    return v;
}

int ensure_ws(frq_device* dev, size_t bytes) {
    if (bytes <= dev->ws_bytes) return FRQ_OK;
    size_t want = bytes < 2 * dev->ws_bytes ? 2 * dev->ws_bytes : bytes;
    if (dev->ws) HIP_TRY(hipFree(dev->ws));  // hipFree waits for work that may use it
    dev->ws = nullptr;
    dev->ws_bytes = 0;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess)
        return fail(FRQ_WORKSPACE, "workspace allocation of %zu bytes failed: %s", want,
                    hipGetErrorString(e));
    dev->ws = p;
    dev->ws_bytes = want;
    return FRQ_OK;
}

int use_device(frq_device* dev) {
    if (!dev) return fail(FRQ_INVALID, "null device handle");
    // HIP keeps the last error of the thread until it is read: drop one left
    // by an earlier call so that the launch checks of this call see their own
    (void)hipGetLastError();
    HIP_TRY(hipSetDevice(dev->ordinal));
    return FRQ_OK;
}

// The device lock for the duration of an entry point (no-op for a null
// handle, which use_device then rejects).
struct DevGuard {
    frq_device* d;
    explicit DevGuard(frq_device* dev) : d(dev) {
        if (d) d->mu.lock();
    }
    ~DevGuard() {
        if (d) d->mu.unlock();
    }
    DevGuard(const DevGuard&) = delete;
    DevGuard& operator=(const DevGuard&) = delete;
};

void release_device(frq_device* dev) {
    if (dev->refs.fetch_sub(1) == 1) delete dev;
}

// Device memory a call may use as scratch: the handle's workspace, grown with
// hipMalloc on demand (base == nullptr), or a fixed region that is never grown
// (the allocation-free entry point's).
struct Scratch {
    uint8_t* base = nullptr;
    size_t bytes = 0;
};

int scratch_at_least(frq_device* dev, const Scratch& fx, size_t bytes, uint8_t** base, const char* who) {
    if (fx.base) {
        if (bytes > fx.bytes)
            return fail(FRQ_WORKSPACE, "%s: needs %zu bytes of scratch; the allocation-free entry point holds %zu",
                        who, bytes, fx.bytes);
        *base = fx.base;
        return FRQ_OK;
    }
    int rc = ensure_ws(dev, bytes);
    if (rc) return rc;
    *base = static_cast<uint8_t*>(dev->ws);
    return FRQ_OK;
}

// Quantize rows x [rows, k] into scratch at `base` (and optionally into fuel's
// block layout at `aos`), returning the view.
int quantize_rows_at(frq_device* dev, int vt, const float* x, size_t rows, size_t k, void* aos, uint8_t* base,
                     ActView* view) {
    *view = act_view(base, vt, rows, k);
    if (rows == 0) return FRQ_OK;
    hipError_t e = vt == GGML_Q8K
                       ? launch_quantize_q8k(x, (int)rows, (int)k, *view, (uint8_t*)aos, dev->stream)
                       : launch_quantize_q8_0(x, (int)rows, (int)k, *view, (uint8_t*)aos, dev->stream);
    HIP_TRY(e);
    return FRQ_OK;
}

// Quantize rows x [rows, k] into the workspace (and optionally into fuel's
// block layout at `aos`), returning the workspace view.
int quantize_rows(frq_device* dev, int vt, const float* x, size_t rows, size_t k, void* aos,
                  ActView* view) {
    int rc = ensure_ws(dev, act_bytes(vt, rows, k));
    if (rc) return rc;
    *view = act_view(dev->ws, vt, rows, k);
    if (rows == 0) return FRQ_OK;
    hipError_t e = vt == GGML_Q8K
                       ? launch_quantize_q8k(x, (int)rows, (int)k, *view, (uint8_t*)aos, dev->stream)
                       : launch_quantize_q8_0(x, (int)rows, (int)k, *view, (uint8_t*)aos, dev->stream);
    HIP_TRY(e);
    return FRQ_OK;
}

// Which kernels a QMatMul of `rows` activation rows runs (frq_qmatmul_plan
// reports it): a pure function of the call's shape, weight type, the weight
// base's 16-byte alignment, the device's CU count and whether the scratch is
// the allocation-free entry point's fixed array -- never of earlier calls.
enum QmmPath { QMM_MATVEC = 0, QMM_MULTI = 1, QMM_SKINNY = 2, QMM_TILED = 3 };

struct QmmPlan {
    int path = QMM_MATVEC;
    MmqPlan mmq{};        // QMM_TILED: kernel kind and K split
    size_t abytes = 0;    // QMM_TILED / QMM_SKINNY: quantized-row scratch bytes
};

int plan_qmatmul(const frq_device* dev, int t, const uint8_t* w, size_t rows, size_t n, size_t k, const Scratch& fx,
                 QmmPlan* p) {
    *p = QmmPlan{};
    if (k > (size_t)0x7fffffff || n > (size_t)0x7fffffff || rows > 65535)
        return fail(FRQ_UNSUPPORTED, "qmatmul: rows=%zu n=%zu k=%zu exceed the launch limits", rows, n, k);
    // each lane of the mat-vec holds at most 8 blocks of a row: K <= 8 * 16 * 256
    // for the k-quants (4 lanes per superblock), K <= 8 * 32 * 32 for Q8_0;
    // longer rows (K a multiple of 256) take the skinny MFMA kernel, any K
    const size_t kmax = t == GGML_Q8_0 ? 8192 : 32768;
    const bool skinny = mmq_skinny_supported(t, (int)k);
    if (k > kmax && !skinny)
        return fail(FRQ_UNSUPPORTED, "qmatmul: k=%zu exceeds %zu for dtype %d", k, kmax, t);
    // the tiled MFMA kernel addresses the weights with 32-bit offsets
    const bool w32 = n * (k / block_elems(t)) * type_size(t) <= 0xffffffffull;
    if (tiled_rows(t, w, rows, n, k) && mmq_supported(t) && w32) {
        // many activation rows: quantize them once, then the int8-MFMA GEMM;
        // scratch: quantized rows, then the split-K partial sums the plan
        // needs (a fixed scratch region lowers the split until they fit)
        p->path = QMM_TILED;
        p->abytes = align256(act_bytes(vec_dot_type(t), rows, k));
        const size_t pcap =
            !fx.base ? ~(size_t)0 : fx.bytes > p->abytes ? (fx.bytes - p->abytes) / sizeof(float) : 0;
        p->mmq = mmq_plan(t, w, (int)rows, (int)n, (int)k, dev->num_cus, pcap);
    } else if (qmv_multi_supported(t, (int)rows, (int)n, (int)k)) {
        // a few rows of the k-quants: the mat-vec with every workgroup
        // quantizing them into LDS, each weight row reduced against all of
        // them (one weight pass per 2 or 4 rows, no quantize launch)
        p->path = QMM_MULTI;
    } else if (skinny && (rows >= 2 || k > kmax)) {
        // a few rows (and Q8_0 at any row count: it has no tiled MFMA
        // kernel): quantize them once, then one weight pass per 32-row group
        p->path = QMM_SKINNY;
        p->abytes = act_bytes(vec_dot_type(t), rows, k);
    } else {
        p->path = QMM_MATVEC;
    }
    return FRQ_OK;
}

// y[rows, n] = x[rows, k] @ dequant(W[n, k])^T through the int8 path, with
// its scratch (quantized rows, split-K partials) from `fx` when that is set.
int run_qmatmul(frq_device* dev, int t, const uint8_t* w, const float* x, size_t rows, size_t n,
                size_t k, float* y, const Scratch& fx = Scratch{}) {
    if (rows == 0 || n == 0) return FRQ_OK;
    QmmPlan plan;
    int rc = plan_qmatmul(dev, t, w, rows, n, k, fx, &plan);
    if (rc) return rc;
    switch (plan.path) {
        case QMM_TILED: {
            uint8_t* base = nullptr;
            rc = scratch_at_least(dev, fx, plan.abytes + plan.mmq.part_elems * sizeof(float), &base, "qmatmul");
            if (rc) return rc;
            ActView act;
            rc = quantize_rows_at(dev, vec_dot_type(t), x, rows, k, nullptr, base, &act);
            if (rc) return rc;
            float* part = plan.mmq.part_elems ? reinterpret_cast<float*>(base + plan.abytes) : nullptr;
            HIP_TRY(launch_mmq(plan.mmq, t, w, act, y, part, (int)rows, (int)n, (int)k, (int)n, dev->stream));
            return FRQ_OK;
        }
        case QMM_MULTI:
            HIP_TRY(launch_qmv_multi(t, w, x, y, (int)rows, (int)n, (int)k, (int)n, dev->stream, dev->num_cus));
            return FRQ_OK;
        case QMM_SKINNY: {
            uint8_t* base = nullptr;
            rc = scratch_at_least(dev, fx, plan.abytes, &base, "qmatmul");
            if (rc) return rc;
            ActView act;
            rc = quantize_rows_at(dev, vec_dot_type(t), x, rows, k, nullptr, base, &act);
            if (rc) return rc;
            HIP_TRY(launch_mmq_skinny(t, w, act, y, (int)rows, (int)n, (int)k, (int)n, dev->num_cus, dev->stream));
            return FRQ_OK;
        }
        default:
            HIP_TRY(launch_qmv(t, w, x, y, (int)rows, (int)n, (int)k, (int)n, dev->stream, dev->num_cus));
            return FRQ_OK;
    }
}

// The batched paths of a fused QMatMul (rows >= 2 formed by a prologue: the
// RMS norm x gain, the SwiGLU product, or a strided row): the rows are formed
// and quantized once (launch_quantize_q8k_src), then the int8-MFMA GEMM (from
// tiled_rows) or the few-row MFMA kernel, the residual added in their
// epilogue when asked (OUT_ACC).  false: no batched path applies (Q8_0
// weights, one row, unsupported K) and the caller runs the fused mat-vec.
struct FusedBatch {
    bool mmq = false;
    MmqPlan plan{};
    size_t abytes = 0;
};

bool fused_batch_plan(frq_device* dev, int t, const void* w, const ActSrc& src, size_t rows, size_t n, size_t k,
                      FusedBatch* fb) {
    if (rows < 2 || vec_dot_type(t) != GGML_Q8K || k > (size_t)0x7fffffff || !quantize_src_supported(src, (int)k))
        return false;
    const bool w32 = n * (k / block_elems(t)) * type_size(t) <= 0xffffffffull;
    if (tiled_rows(t, w, rows, n, k) && mmq_supported(t) && w32) {
        fb->mmq = true;
        fb->plan = mmq_plan(t, w, (int)rows, (int)n, (int)k, dev->num_cus);
    } else if (mmq_skinny_supported(t, (int)k)) {
        fb->mmq = false;
        fb->plan = MmqPlan{};
    } else {
        return false;
    }
    fb->abytes = align256(act_bytes(GGML_Q8K, rows, k));
    return true;
}

hipError_t launch_fused_batch(frq_device* dev, const FusedBatch& fb, int t, const void* w, const ActView& act,
                              size_t rows, size_t n, size_t k, float* y, size_t ldy, int out_mode) {
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (fb.mmq) {
        float* part = fb.plan.part_elems ? reinterpret_cast<float*>(static_cast<uint8_t*>(dev->ws) + fb.abytes) : nullptr;
        return launch_mmq(fb.plan, t, wb, act, y, part, (int)rows, (int)n, (int)k, (int)ldy, dev->stream, out_mode);
    }
    return launch_mmq_skinny(t, wb, act, y, (int)rows, (int)n, (int)k, (int)ldy, dev->num_cus, dev->stream, out_mode);
}

// matmul_f16 (k_quants.rs:2333-2374): f16 rows x [rows, k] widened exactly to
// f32, then the same quantize and block dots as run_qmatmul; each f32 output
// is rounded to f16 (f16::from_f32, nearest even) as it is stored.
int run_qmatmul_f16(frq_device* dev, int t, const uint8_t* w, const uint16_t* x, size_t rows, size_t n, size_t k,
                    uint16_t* y) {
    if (rows == 0 || n == 0) return FRQ_OK;
    if (k > (size_t)0x7fffffff || n > (size_t)0x7fffffff || rows > 65535)
        return fail(FRQ_UNSUPPORTED, "qmatmul_f16: rows=%zu n=%zu k=%zu exceed the launch limits", rows, n, k);
    // the same kernels as run_qmatmul for the same rows (so that the outputs
    // are the f32 path's, rounded), with f16 activation loads and stores
    const size_t kmax = t == GGML_Q8_0 ? 8192 : 32768;
    const bool skinny = mmq_skinny_supported(t, (int)k);
    if (k > kmax && !skinny)
        return fail(FRQ_UNSUPPORTED, "qmatmul_f16: k=%zu exceeds %zu for dtype %d", k, kmax, t);
    const bool w32 = n * (k / block_elems(t)) * type_size(t) <= 0xffffffffull;
    if (tiled_rows(t, w, rows, n, k) && mmq_supported(t) && w32) {
        const MmqPlan plan = mmq_plan(t, w, (int)rows, (int)n, (int)k, dev->num_cus);
        const size_t abytes = align256(act_bytes(GGML_Q8K, rows, k));
        int rc = ensure_ws(dev, abytes + plan.part_elems * sizeof(float));
        if (rc) return rc;
        const ActView act = act_view(dev->ws, GGML_Q8K, rows, k);
        HIP_TRY(launch_quantize_q8k_h(x, (int)rows, (int)k, act, dev->stream));
        float* part = plan.part_elems ? reinterpret_cast<float*>(static_cast<uint8_t*>(dev->ws) + abytes) : nullptr;
        HIP_TRY(launch_mmq(plan, t, w, act, reinterpret_cast<float*>(y), part, (int)rows, (int)n, (int)k, (int)n,
                           dev->stream, true));
        return FRQ_OK;
    }
    if (skinny && (rows >= 2 || k > kmax)) {
        const int vt = vec_dot_type(t);
        int rc = ensure_ws(dev, act_bytes(vt, rows, k));
        if (rc) return rc;
        const ActView act = act_view(dev->ws, vt, rows, k);
        HIP_TRY(vt == GGML_Q8K ? launch_quantize_q8k_h(x, (int)rows, (int)k, act, dev->stream)
                               : launch_quantize_q8_0_h(x, (int)rows, (int)k, act, dev->stream));
        HIP_TRY(launch_mmq_skinny(t, w, act, reinterpret_cast<float*>(y), (int)rows, (int)n, (int)k, (int)n,
                                  dev->num_cus, dev->stream, true));
        return FRQ_OK;
    }
    HIP_TRY(launch_qmv_half(t, w, x, y, (int)rows, (int)n, (int)k, (int)n, dev->stream, dev->num_cus));
    return FRQ_OK;
}

bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }

// Largest K a mat-vec lane group covers (8 register slots per lane).
size_t qmv_kmax(int t) { return t == GGML_Q8_0 ? 8192 : 32768; }

// Indexed mat-vec over M launch rows, in launches of at most 65535 rows (the
// grid's y limit).  With a null x_row the activation row is m / x_div, so the
// chunks hold whole multiples of x_div rows.
int run_indexed(frq_device* dev, int t, const uint8_t* w, const float* x, size_t M, int N, int K, float* y, int ldy,
                QmvOpts ix) {
    const size_t step = ix.x_row ? 65535 : (size_t)(65535 / ix.x_div) * ix.x_div;
    for (size_t m0 = 0; m0 < M; m0 += step) {
        const size_t rows = M - m0 < step ? M - m0 : step;
        QmvOpts c = ix;
        const float* xc = x;
        c.w_sel = ix.w_sel ? ix.w_sel + m0 : nullptr;
        if (ix.route_logits) {  // rows m0.. start on a token boundary (step is a multiple of x_div)
            c.route_logits = ix.route_logits + m0 / ix.x_div * (size_t)ix.n_experts;
            c.route_ids = ix.route_ids + m0;
            c.route_w = ix.route_w + m0;
        }
        if (ix.x_row) {
            c.x_row = ix.x_row + m0;
        } else {
            const size_t xo = m0 / ix.x_div * (size_t)ix.ldx;
            xc = x + xo;
            if (ix.x2) c.x2 = ix.x2 + xo;
        }
        if (ix.route_logits)
            HIP_TRY(launch_qmv_indexed_route(t, w, xc, y + m0 * (size_t)ldy, (int)rows, N, K, ldy, c, dev->stream,
                                             dev->num_cus));
        else
            HIP_TRY(launch_qmv_indexed(t, w, xc, y + m0 * (size_t)ldy, (int)rows, N, K, ldy, c, dev->stream,
                                       dev->num_cus));
    }
    return FRQ_OK;
}

int check_moe_dims(const char* who, size_t e, size_t topk) {
    if (e == 0 || e > (size_t)MOE_MAX_EXPERTS)
        return fail(FRQ_UNSUPPORTED, "%s: %zu experts (supported 1..%d)", who, e, MOE_MAX_EXPERTS);
    if (topk == 0 || topk > e || topk > (size_t)MOE_MAX_TOPK)
        return fail(FRQ_INVALID, "%s: topk=%zu must be in 1..min(experts=%zu, %d)", who, topk, e, MOE_MAX_TOPK);
    return FRQ_OK;
}

// Routing + expert batches into caller buffers; entry_expert / entry_pos are
// device scratch of t * topk ints.
int route_and_batch(frq_device* dev, const float* logits, size_t t, size_t e, size_t topk, int* ids, float* w,
                    int* offsets, int* sorted_token, int* sorted_slot, int* entry_expert, int* entry_pos,
                    const MoeTiles& tiles = MoeTiles{}) {
    HIP_TRY(launch_moe_route(logits, (int)t, (int)e, (int)topk, ids, w, dev->stream));
    HIP_TRY(launch_moe_batches(ids, (int)(t * topk), (int)e, (int)topk, offsets, sorted_token, sorted_slot,
                               entry_expert, entry_pos, tiles, dev->stream));
    return FRQ_OK;
}

// Beyond this many routed entries per expert on average, the expert
// projections run as grouped int8-MFMA matmuls (one weight pass per expert
// tile) instead of one mat-vec per routed row (Qwen3-MoE layer, 128 experts:
// the mat-vec wins at 128 entries, 72 against 81 us; the grouped tiles from
// 160 entries, 85 against 89 us).
constexpr double MOE_MMQ_MIN_ROWS_PER_EXPERT = 1.0;

}  // namespace

extern "C" {

const char* frq_last_error(void) { return g_err.c_str(); }

size_t frq_type_size(int t) { return type_size(t); }
size_t frq_block_size(int t) { return block_elems(t); }

int frq_device_count(int* count) {
    if (!count) return fail(FRQ_INVALID, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return FRQ_OK;
}

int frq_device_open(int ordinal, frq_device** out) {
    if (!out) return fail(FRQ_INVALID, "null out");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || ordinal < 0 || ordinal >= n)
        return fail(FRQ_INVALID, "device ordinal %d not present (%d devices)", ordinal, n);
    HIP_TRY(hipSetDevice(ordinal));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, ordinal));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(FRQ_UNSUPPORTED, "device %d is %s; this library is built for gfx950", ordinal,
                    prop.gcnArchName);
    // this device's copy of the allocation-free entry point's scratch array
    // (looked up with the device current)
    void* sp = nullptr;
    HIP_TRY(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
    if (!sp) return fail(FRQ_INTERNAL, "hipGetSymbolAddress(scratch) returned a null address on device %d", ordinal);
    frq_device* d = new frq_device();
    d->ordinal = ordinal;
    d->num_cus = prop.multiProcessorCount;
    d->scratch = sp;
    hipError_t e = hipStreamCreateWithFlags(&d->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete d;
        return fail(FRQ_INTERNAL, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    d->stream = d->own_stream;
    *out = d;
    return FRQ_OK;
}

int frq_device_close(frq_device* dev) {
    if (!dev) return FRQ_OK;
    {
        DevGuard guard(dev);
        (void)hipSetDevice(dev->ordinal);
        (void)hipStreamSynchronize(dev->stream);
        if (dev->ws) (void)hipFree(dev->ws);
        dev->ws = nullptr;
        dev->ws_bytes = 0;
        if (dev->own_stream) (void)hipStreamDestroy(dev->own_stream);
        dev->own_stream = dev->stream = nullptr;
        (void)hipGetLastError();
    }
    release_device(dev);  // storages still alive keep the struct until they are freed
    return FRQ_OK;
}

int frq_device_set_stream(frq_device* dev, void* s) {
    if (!dev) return fail(FRQ_INVALID, "null device");
    DevGuard guard(dev);
    dev->stream = s ? static_cast<hipStream_t>(s) : dev->own_stream;
    return FRQ_OK;
}

int frq_sync(frq_device* dev) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return FRQ_OK;
}

int frq_device_cu_count(const frq_device* dev, int* cus) {
    if (!dev || !cus) return fail(FRQ_INVALID, "null argument");
    *cus = dev->num_cus;
    return FRQ_OK;
}

int frq_device_workspace_bytes(const frq_device* dev, size_t* bytes) {
    if (!dev || !bytes) return fail(FRQ_INVALID, "null argument");
    DevGuard guard(const_cast<frq_device*>(dev));
    *bytes = dev->ws_bytes;
    return FRQ_OK;
}

int frq_malloc(frq_device* dev, size_t bytes, void** dptr) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!dptr) return fail(FRQ_INVALID, "null out");
    *dptr = nullptr;
    if (bytes == 0) return FRQ_OK;
    hipError_t e = hipMalloc(dptr, bytes);
    if (e != hipSuccess) return fail(FRQ_WORKSPACE, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return FRQ_OK;
}

int frq_free(frq_device* dev, void* p) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (p) HIP_TRY(hipFree(p));
    return FRQ_OK;
}

int frq_memcpy_htod(frq_device* dev, void* dst, const void* src, size_t bytes) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!bytes) return FRQ_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return FRQ_OK;
}

int frq_memcpy_dtoh(frq_device* dev, void* dst, const void* src, size_t bytes) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!bytes) return FRQ_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return FRQ_OK;
}

int frq_memcpy_dtod(frq_device* dev, void* dst, const void* src, size_t bytes) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!bytes) return FRQ_OK;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, dev->stream));
    return FRQ_OK;
}

int frq_memset(frq_device* dev, void* dst, int value, size_t bytes) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!bytes) return FRQ_OK;
    HIP_TRY(hipMemsetAsync(dst, value, bytes, dev->stream));
    return FRQ_OK;
}

// ---- QuantizedDeviceKernels ----

static int new_storage(frq_device* dev, int t, size_t nbytes, frq_qstorage** out) {
    frq_qstorage* q = new frq_qstorage();
    q->dev = dev;
    q->dtype = t;
    q->nbytes = nbytes;
    if (nbytes) {
        hipError_t e = hipMalloc(&q->d_ptr, nbytes);
        if (e != hipSuccess) {
            delete q;
            return fail(FRQ_WORKSPACE, "hipMalloc(%zu): %s", nbytes, hipGetErrorString(e));
        }
    }
    dev->refs.fetch_add(1);
    *out = q;
    return FRQ_OK;
}

int frq_qstorage_zeros(frq_device* dev, int t, size_t elem_count, frq_qstorage** out) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!out) return fail(FRQ_INVALID, "null out");
    if (!type_size(t)) return fail(FRQ_UNSUPPORTED, "qzeros: unsupported dtype %d", t);
    if (elem_count % block_elems(t))
        return fail(FRQ_INVALID, "qzeros: elem_count %zu is not a multiple of %zu", elem_count,
                    block_elems(t));
    const size_t nbytes = elem_count / block_elems(t) * type_size(t);
    rc = new_storage(dev, t, nbytes, out);
    if (rc) return rc;
    if (nbytes) HIP_TRY(hipMemsetAsync((*out)->d_ptr, 0, nbytes, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return FRQ_OK;
}

int frq_qstorage_load(frq_device* dev, int t, const void* host, size_t nbytes, frq_qstorage** out) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!out) return fail(FRQ_INVALID, "null out");
    if (!type_size(t)) return fail(FRQ_UNSUPPORTED, "load_quantized: unsupported dtype %d", t);
    if (nbytes % type_size(t))
        return fail(FRQ_INVALID, "load_quantized: %zu bytes is not a multiple of the %zu-byte block",
                    nbytes, type_size(t));
    if (nbytes && !host) return fail(FRQ_INVALID, "load_quantized: null host data");
    rc = new_storage(dev, t, nbytes, out);
    if (rc) return rc;
    if (nbytes) {
        HIP_TRY(hipMemcpyAsync((*out)->d_ptr, host, nbytes, hipMemcpyHostToDevice, dev->stream));
        HIP_TRY(hipStreamSynchronize(dev->stream));
    }
    return FRQ_OK;
}

int frq_qstorage_free(frq_qstorage* q) {
    if (!q) return FRQ_OK;
    if (q->d_ptr) {
        (void)hipSetDevice(q->dev->ordinal);
        (void)hipFree(q->d_ptr);  // waits for work that may still use the blocks
        (void)hipGetLastError();
    }
    release_device(q->dev);
    delete q;
    return FRQ_OK;
}

// ---- DynQuantizedStorage ----

int frq_qstorage_dtype(const frq_qstorage* q) { return q ? q->dtype : -1; }
size_t frq_qstorage_block_size(const frq_qstorage* q) { return q ? block_elems(q->dtype) : 0; }
size_t frq_qstorage_size_in_bytes(const frq_qstorage* q) { return q ? q->nbytes : 0; }

int frq_qstorage_data(const frq_qstorage* q, void* host, size_t nbytes) {
    if (!q) return fail(FRQ_INVALID, "null storage");
    if (nbytes != q->nbytes) return fail(FRQ_INVALID, "data: buffer %zu bytes, storage %zu", nbytes, q->nbytes);
    return frq_memcpy_dtoh(q->dev, host, q->d_ptr, nbytes);
}

int frq_qstorage_device_ptr(const frq_qstorage* q, const void** out) {
    if (!q || !out) return fail(FRQ_INVALID, "null argument");
    *out = q->d_ptr;
    return FRQ_OK;
}

static int dequant_common(const frq_qstorage* q, size_t elem_count, void* y, bool f16) {
    if (!q) return fail(FRQ_INVALID, "null storage");
    DevGuard guard(q->dev);
    int rc = use_device(q->dev);
    if (rc) return rc;
    if (!is_weight_type(q->dtype)) return fail(FRQ_UNSUPPORTED, "dequantize: dtype %d", q->dtype);
    const size_t blocks = q->nbytes / type_size(q->dtype);
    if (elem_count != blocks * block_elems(q->dtype))
        return fail(FRQ_INVALID, "dequantize: elem_count %zu but storage holds %zu", elem_count,
                    blocks * block_elems(q->dtype));
    if (!aligned4(y) && !f16) return fail(FRQ_MISALIGNED, "dequantize: output not 4-byte aligned");
    HIP_TRY(launch_dequantize(q->dtype, q->d_ptr, blocks, (float*)y, f16, q->dev->stream));
    return FRQ_OK;
}

int frq_qstorage_dequantize(const frq_qstorage* q, size_t elem_count, float* y) {
    return dequant_common(q, elem_count, y, false);
}

int frq_qstorage_dequantize_f16(const frq_qstorage* q, size_t elem_count, uint16_t* y) {
    return dequant_common(q, elem_count, y, true);
}

int frq_qstorage_quantize(frq_qstorage* q, const float* src, size_t elem_count) {
    if (!q) return fail(FRQ_INVALID, "null storage");
    DevGuard guard(q->dev);
    int rc = use_device(q->dev);
    if (rc) return rc;
    if (!is_weight_type(q->dtype)) return fail(FRQ_UNSUPPORTED, "quantize: dtype %d", q->dtype);
    const size_t blocks = q->nbytes / type_size(q->dtype);
    if (elem_count != blocks * block_elems(q->dtype))
        return fail(FRQ_INVALID, "quantize: %zu source elements for a storage of %zu", elem_count,
                    blocks * block_elems(q->dtype));
    if (((uintptr_t)src & 15u) != 0) return fail(FRQ_MISALIGNED, "quantize: source must be 16-byte aligned");
    HIP_TRY(launch_quantize_weights(q->dtype, src, blocks, q->d_ptr, q->dev->stream));
    return FRQ_OK;
}

int frq_qstorage_quantize_imatrix(frq_qstorage* q, const float* src, size_t elem_count, const float* imatrix,
                                  size_t n_per_row) {
    if (!q) return fail(FRQ_INVALID, "null storage");
    DevGuard guard(q->dev);
    int rc = use_device(q->dev);
    if (rc) return rc;
    if (q->dtype != GGML_Q4K && q->dtype != GGML_Q6K)
        return fail(FRQ_UNSUPPORTED, "quantize_imatrix: from_float_imatrix is not implemented for dtype %d", q->dtype);
    const size_t blocks = q->nbytes / type_size(q->dtype);
    if (elem_count != blocks * QK_K)
        return fail(FRQ_INVALID, "quantize_imatrix: %zu source elements for a storage of %zu", elem_count,
                    blocks * (size_t)QK_K);
    if (n_per_row == 0 || n_per_row % QK_K)
        return fail(FRQ_INVALID, "quantize_imatrix: n_per_row=%zu must be a positive multiple of %d", n_per_row, QK_K);
    if (!imatrix || (elem_count && !src)) return fail(FRQ_INVALID, "quantize_imatrix: null buffer");
    if (((uintptr_t)src & 15u) != 0) return fail(FRQ_MISALIGNED, "quantize_imatrix: source must be 16-byte aligned");
    if (blocks == 0) return FRQ_OK;
    // the importance weights go to the workspace (stream-ordered before the kernel)
    if ((rc = ensure_ws(q->dev, n_per_row * sizeof(float)))) return rc;
    float* wdev = static_cast<float*>(q->dev->ws);
    HIP_TRY(hipMemcpyAsync(wdev, imatrix, n_per_row * sizeof(float), hipMemcpyHostToDevice, q->dev->stream));
    HIP_TRY(launch_quantize_weights_imatrix(q->dtype, src, blocks, wdev, n_per_row / QK_K, q->d_ptr,
                                            q->dev->stream));
    // the host buffer may be reused once this returns: wait for the copy
    HIP_TRY(hipStreamSynchronize(q->dev->stream));
    return FRQ_OK;
}

int frq_qstorage_fwd(const frq_qstorage* q, size_t n, size_t k, const float* x, size_t m, float* y) {
    if (!q) return fail(FRQ_INVALID, "null storage");
    DevGuard guard(q->dev);
    int rc = use_device(q->dev);
    if (rc) return rc;
    if (!is_weight_type(q->dtype)) return fail(FRQ_UNSUPPORTED, "fwd: dtype %d", q->dtype);
    if (k % block_elems(q->dtype))
        return fail(FRQ_INVALID, "fwd: k=%zu is not a multiple of %zu", k, block_elems(q->dtype));
    if (n * (k / block_elems(q->dtype)) * type_size(q->dtype) != q->nbytes)
        return fail(FRQ_INVALID, "fwd: shape [%zu, %zu] does not match %zu storage bytes", n, k,
                    q->nbytes);
    if (!aligned4(x) || !aligned4(y)) return fail(FRQ_MISALIGNED, "fwd: f32 buffers must be 4-byte aligned");
    return run_qmatmul(q->dev, q->dtype, q->d_ptr, x, m, n, k, y);
}

int frq_qstorage_fwd_f16(const frq_qstorage* q, size_t n, size_t k, const uint16_t* x, size_t m, uint16_t* y) {
    if (!q) return fail(FRQ_INVALID, "null storage");
    DevGuard guard(q->dev);
    int rc = use_device(q->dev);
    if (rc) return rc;
    if (!is_weight_type(q->dtype)) return fail(FRQ_UNSUPPORTED, "fwd_f16: dtype %d", q->dtype);
    if (k % block_elems(q->dtype))
        return fail(FRQ_INVALID, "fwd_f16: k=%zu is not a multiple of %zu", k, block_elems(q->dtype));
    if (n * (k / block_elems(q->dtype)) * type_size(q->dtype) != q->nbytes)
        return fail(FRQ_INVALID, "fwd_f16: shape [%zu, %zu] does not match %zu storage bytes", n, k, q->nbytes);
    // rows are read 4 halves (8 bytes) per lane: k is a multiple of 32, so 8-byte alignment of x suffices
    if (((uintptr_t)x & 7u) != 0 || ((uintptr_t)y & 1u) != 0)
        return fail(FRQ_MISALIGNED, "fwd_f16: x must be 8-byte and y 2-byte aligned");
    return run_qmatmul_f16(q->dev, q->dtype, q->d_ptr, x, m, n, k, y);
}

// ---- KernelRef seam ----

namespace {

// frq_qmatmul's checks (qmatmul_generic_f32, byte_kernels.rs:4767-4806), then
// the matmul with its scratch from `fx` when set.
int qmatmul_checked(frq_device* dev, int t, size_t batch, size_t m, size_t n, size_t k, const float* act,
                    size_t act_b, const uint32_t* w, size_t w_b, float* out, size_t out_b, const Scratch& fx) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!is_weight_type(t)) return fail(FRQ_UNSUPPORTED, "qmatmul: unsupported quant_type %d", t);
    const size_t bs = block_elems(t);
    if (k % bs) return fail(FRQ_INVALID, "qmatmul: k=%zu must be a multiple of block size %zu", k, bs);
    const size_t need_w = n * (k / bs) * type_size(t);
    const size_t need_a = batch * m * k * sizeof(float);
    const size_t need_o = batch * m * n * sizeof(float);
    if (act_b != need_a)
        return fail(FRQ_INVALID, "qmatmul: activations bytes=%zu doesn't match batch=%zu x m=%zu x k=%zu x 4",
                    act_b, batch, m, k);
    if (w_b != need_w)
        return fail(FRQ_INVALID, "qmatmul: weight bytes=%zu doesn't match n=%zu x k/block_size=%zu x %zu",
                    w_b, n, k / bs, type_size(t));
    if (out_b != need_o)
        return fail(FRQ_INVALID, "qmatmul: out bytes=%zu doesn't match batch=%zu x m=%zu x n=%zu x 4",
                    out_b, batch, m, n);
    if (batch == 0 || m == 0 || n == 0) return FRQ_OK;
    if (!aligned4(w) || !aligned4(act) || !aligned4(out))
        return fail(FRQ_MISALIGNED, "qmatmul: buffers must be 4-byte aligned");
    // The batch shares W, so all batch*m activation rows go through one launch.
    return run_qmatmul(dev, t, reinterpret_cast<const uint8_t*>(w), act, batch * m, n, k, out, fx);
}

}  // namespace

int frq_qmatmul(frq_device* dev, int t, size_t batch, size_t m, size_t n, size_t k, const float* act,
                size_t act_b, const uint32_t* w, size_t w_b, float* out, size_t out_b) {
    return qmatmul_checked(dev, t, batch, m, n, k, act, act_b, w, w_b, out, out_b, Scratch{});
}

int frq_qmatmul_noalloc(frq_device* dev, int t, size_t batch, size_t m, size_t n, size_t k, const float* act,
                        size_t act_b, const uint32_t* w, size_t w_b, float* out, size_t out_b) {
    if (!dev) return fail(FRQ_INVALID, "null device handle");
    Scratch fx;
    fx.base = static_cast<uint8_t*>(dev->scratch);
    fx.bytes = FRQ_NOALLOC_SCRATCH_BYTES;
    return qmatmul_checked(dev, t, batch, m, n, k, act, act_b, w, w_b, out, out_b, fx);
}

int frq_qmatmul_plan(frq_device* dev, int t, size_t rows, size_t n, size_t k, const void* w, int noalloc, int* path,
                     int* kind, int* ksplit) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!path || !kind || !ksplit) return fail(FRQ_INVALID, "qmatmul_plan: null output");
    if (!is_weight_type(t)) return fail(FRQ_UNSUPPORTED, "qmatmul_plan: unsupported quant_type %d", t);
    if (k % block_elems(t)) return fail(FRQ_INVALID, "qmatmul_plan: k=%zu must be a multiple of %zu", k, block_elems(t));
    Scratch fx;
    if (noalloc) {
        fx.base = static_cast<uint8_t*>(dev->scratch);
        fx.bytes = FRQ_NOALLOC_SCRATCH_BYTES;
    }
    QmmPlan p;
    if ((rc = plan_qmatmul(dev, t, static_cast<const uint8_t*>(w), rows, n, k, fx, &p))) return rc;
    *path = p.path;
    *kind = p.path == QMM_TILED ? p.mmq.kind : -1;
    *ksplit = p.path == QMM_TILED ? (p.mmq.ks > 1 ? p.mmq.ks : 1) : 1;
    return FRQ_OK;
}

// ---- taps ----

int frq_quantize_q8k(frq_device* dev, const float* x, size_t rows, size_t k, void* blocks) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (k % QK_K) return fail(FRQ_INVALID, "quantize_q8k: k=%zu not a multiple of 256", k);
    if (rows > 65535) return fail(FRQ_UNSUPPORTED, "quantize_q8k: rows=%zu", rows);
    ActView v;
    return quantize_rows(dev, GGML_Q8K, x, rows, k, blocks, &v);
}

int frq_quantize_q8_0(frq_device* dev, const float* x, size_t rows, size_t k, void* blocks) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (k % QK8_0) return fail(FRQ_INVALID, "quantize_q8_0: k=%zu not a multiple of 32", k);
    if (rows > 65535) return fail(FRQ_UNSUPPORTED, "quantize_q8_0: rows=%zu", rows);
    ActView v;
    return quantize_rows(dev, GGML_Q8_0, x, rows, k, blocks, &v);
}

int frq_block_isums(frq_device* dev, int t, size_t m, size_t n, size_t k, const void* w,
                    const float* x, int32_t* isum, int32_t* msum) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!is_weight_type(t)) return fail(FRQ_UNSUPPORTED, "block_isums: dtype %d", t);
    if (k % block_elems(t)) return fail(FRQ_INVALID, "block_isums: k=%zu", k);
    if (m > 65535) return fail(FRQ_UNSUPPORTED, "block_isums: m=%zu", m);
    if (m == 0 || n == 0) return FRQ_OK;
    ActView act;
    rc = quantize_rows(dev, vec_dot_type(t), x, m, k, nullptr, &act);
    if (rc) return rc;
    HIP_TRY(launch_block_isums(t, (const uint8_t*)w, act, isum, msum, (int)m, (int)n, (int)k, dev->stream));
    return FRQ_OK;
}

// ---- MoE ----

int frq_moe_route(frq_device* dev, const float* logits, size_t t, size_t e, size_t topk, int32_t* ids, float* w,
                  int32_t* offsets, int32_t* sorted_token, int32_t* sorted_slot) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if ((rc = check_moe_dims("moe_route", e, topk))) return rc;
    if (t * topk > (size_t)0x7fffffff) return fail(FRQ_UNSUPPORTED, "moe_route: t=%zu too large", t);
    if (!logits || !ids || !w || !offsets || !sorted_token) return fail(FRQ_INVALID, "moe_route: null buffer");
    if (t == 0) {
        HIP_TRY(hipMemsetAsync(offsets, 0, (e + 1) * sizeof(int32_t), dev->stream));
        return FRQ_OK;
    }
    const size_t p = t * topk;
    if ((rc = ensure_ws(dev, 2 * align256(p * sizeof(int))))) return rc;
    int* entry_expert = static_cast<int*>(dev->ws);
    int* entry_pos = reinterpret_cast<int*>(static_cast<uint8_t*>(dev->ws) + align256(p * sizeof(int)));
    return route_and_batch(dev, logits, t, e, topk, ids, w, offsets, sorted_token, sorted_slot, entry_expert,
                           entry_pos);
}

int frq_indexed_moe_forward(const frq_qstorage* q, size_t e, size_t n, size_t k, const float* x, size_t t,
                            size_t x_slots, const int32_t* ids, size_t topk, float* y) {
    if (!q) return fail(FRQ_INVALID, "null storage");
    DevGuard guard(q->dev);
    int rc = use_device(q->dev);
    if (rc) return rc;
    const int dt = q->dtype;
    if (!is_weight_type(dt)) return fail(FRQ_UNSUPPORTED, "indexed_moe_forward: dtype %d", dt);
    if (k % block_elems(dt))
        return fail(FRQ_INVALID, "indexed_moe_forward: k=%zu is not a multiple of %zu", k, block_elems(dt));
    const size_t expert_bytes = n * (k / block_elems(dt)) * type_size(dt);
    if (e * expert_bytes != q->nbytes)
        return fail(FRQ_INVALID, "indexed_moe_forward: shape [%zu, %zu, %zu] does not match %zu storage bytes", e, n,
                    k, q->nbytes);
    if (topk == 0 || topk > 65535) return fail(FRQ_INVALID, "indexed_moe_forward: topk=%zu", topk);
    if (x_slots != 1 && x_slots != topk)
        return fail(FRQ_INVALID, "indexed_moe_forward: input has %zu rows per token, expected 1 or topk=%zu", x_slots,
                    topk);
    if (k > qmv_kmax(dt)) return fail(FRQ_UNSUPPORTED, "indexed_moe_forward: k=%zu exceeds %zu", k, qmv_kmax(dt));
    if (n > (size_t)0x7fffffff || t * topk > (size_t)0x7fffffff || e > (size_t)0x7fffffff)
        return fail(FRQ_UNSUPPORTED, "indexed_moe_forward: sizes exceed the launch limits");
    if (t == 0 || n == 0) return FRQ_OK;
    if (!x || !ids || !y) return fail(FRQ_INVALID, "indexed_moe_forward: null buffer");
    if (!aligned4(x) || !aligned4(y)) return fail(FRQ_MISALIGNED, "indexed_moe_forward: f32 buffers not 4-byte aligned");
    QmvOpts ix{};
    ix.x_row = nullptr;
    ix.x_div = x_slots == 1 ? (int)topk : 1;
    ix.ldx = (int)k;
    ix.w_sel = ids;
    ix.n_experts = (int)e;
    ix.expert_bytes = expert_bytes;
    return run_indexed(q->dev, dt, q->d_ptr, x, t * topk, (int)n, (int)k, y, (int)n, ix);
}

int frq_moe_ffn(frq_device* dev, int dt, size_t t, size_t d, size_t ffn, size_t e, size_t topk, const float* x,
                const float* logits, const void* w_gate, const void* w_up, const void* w_down, float* out) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!is_weight_type(dt)) return fail(FRQ_UNSUPPORTED, "moe_ffn: dtype %d", dt);
    if ((rc = check_moe_dims("moe_ffn", e, topk))) return rc;
    const size_t bs = block_elems(dt);
    if (d % bs || ffn % bs || d == 0 || ffn == 0)
        return fail(FRQ_INVALID, "moe_ffn: d=%zu and ffn=%zu must be positive multiples of %zu", d, ffn, bs);
    if (d > qmv_kmax(dt) || ffn > qmv_kmax(dt))
        return fail(FRQ_UNSUPPORTED, "moe_ffn: d=%zu / ffn=%zu exceed %zu", d, ffn, qmv_kmax(dt));
    if (t * topk > (size_t)0x7fffffff / (2 * ffn > d ? 2 * ffn : d))
        return fail(FRQ_UNSUPPORTED, "moe_ffn: t=%zu too large", t);
    if (t == 0) return FRQ_OK;
    if (!x || !logits || !w_gate || !w_up || !w_down || !out) return fail(FRQ_INVALID, "moe_ffn: null buffer");
    if (!aligned4(x) || !aligned4(out) || !aligned4(logits))
        return fail(FRQ_MISALIGNED, "moe_ffn: f32 buffers not 4-byte aligned");
    const size_t p = t * topk;
    const bool grouped = mmq_supported(dt) && (double)p > MOE_MMQ_MIN_ROWS_PER_EXPERT * (double)e;
    const int bm = mmq_group_rows((int)(p / e));
    const size_t max_tiles = grouped ? (p + bm - 1) / bm + e : 0;
    // workspace: ids, w, sorted token, entry expert, entry position, offsets,
    // tile table, gate|up outputs [p, 2 ffn], down outputs [p, d], and for the
    // grouped path the quantized x [t, d] and silu(gate) * up [p, ffn] rows
    const size_t ib = align256(p * sizeof(int));
    const size_t ob = align256((e + 1) * sizeof(int));
    const size_t tb = align256((max_tiles + 1) * sizeof(int));
    const size_t gub = align256(p * 2 * ffn * sizeof(float));
    const size_t ydb = align256(p * d * sizeof(float));
    const size_t axb = grouped ? align256(act_bytes(GGML_Q8K, t, d)) : 0;
    const size_t ahb = grouped ? align256(act_bytes(GGML_Q8K, p, ffn)) : 0;
    if ((rc = ensure_ws(dev, 5 * ib + ob + 3 * tb + gub + ydb + axb + ahb))) return rc;
    uint8_t* b = static_cast<uint8_t*>(dev->ws);
    auto carve = [&b](size_t n) {
        uint8_t* r = b;
        b += n;
        return r;
    };
    int* ids = reinterpret_cast<int*>(carve(ib));
    float* wts = reinterpret_cast<float*>(carve(ib));
    int* sorted_token = reinterpret_cast<int*>(carve(ib));
    int* entry_expert = reinterpret_cast<int*>(carve(ib));
    int* entry_pos = reinterpret_cast<int*>(carve(ib));
    int* offsets = reinterpret_cast<int*>(carve(ob));
    MoeTiles tiles{};
    tiles.bm = grouped ? bm : 0;
    tiles.tile_expert = reinterpret_cast<int*>(carve(tb));
    tiles.tile_row0 = reinterpret_cast<int*>(carve(tb));
    tiles.ntiles = reinterpret_cast<int*>(carve(tb));
    float* gu = reinterpret_cast<float*>(carve(gub));
    float* yd = reinterpret_cast<float*>(carve(ydb));
    void* ax = carve(axb);
    void* ah = carve(ahb);
    // The grouped path needs the expert batches; the mat-vec path takes its
    // launch rows in (token, slot) order straight from the routing, and the
    // combine still sums each token's entries in ascending expert order.
    if (grouped) {
        if ((rc = route_and_batch(dev, logits, t, e, topk, ids, wts, offsets, sorted_token, nullptr, entry_expert,
                                  entry_pos, tiles)))
            return rc;
    } else if (e > (size_t)QMV_ROUTE_MAX_EXPERTS) {  // (with fewer experts the gate|up launch routes)
        HIP_TRY(launch_moe_route(logits, (int)t, (int)e, (int)topk, ids, wts, dev->stream));
    }
    const size_t gate_bytes = ffn * (d / bs) * type_size(dt);
    const size_t down_bytes = d * (ffn / bs) * type_size(dt);
    if (grouped) {
        // x rows quantized once; the gate|up tiles gather them by token
        const ActView xv = act_view(ax, GGML_Q8K, t, d);
        HIP_TRY(launch_quantize_q8k(x, (int)t, (int)d, xv, nullptr, dev->stream));
        MmqGroup g{};
        g.tile_expert = tiles.tile_expert;
        g.tile_row0 = tiles.tile_row0;
        g.ntiles = tiles.ntiles;
        g.expert_offsets = offsets;
        g.x_row = sorted_token;
        g.expert_bytes = gate_bytes;
        g.w2 = static_cast<const uint8_t*>(w_up);
        g.n_split = (int)ffn;
        HIP_TRY(launch_mmq_grouped(dt, static_cast<const uint8_t*>(w_gate), xv, gu, bm, (int)max_tiles,
                                   (int)(2 * ffn), (int)d, (int)(2 * ffn), g, dev->stream));
        // silu(gate) * up quantized per sorted row, then the down tiles
        const ActView hv = act_view(ah, GGML_Q8K, p, ffn);
        HIP_TRY(launch_quantize_q8k_swiglu(gu, (int)(2 * ffn), (int)p, (int)ffn, hv, dev->stream));
        g.x_row = nullptr;
        g.expert_bytes = down_bytes;
        g.w2 = nullptr;
        g.n_split = 0;
        HIP_TRY(launch_mmq_grouped(dt, static_cast<const uint8_t*>(w_down), hv, yd, bm, (int)max_tiles, (int)d,
                                   (int)ffn, (int)d, g, dev->stream));
        HIP_TRY(launch_moe_combine(yd, ids, wts, entry_pos, (int)t, (int)topk, (int)d, out, dev->stream));
        return FRQ_OK;
    }
    // gate | up in one launch over the entries: gu[p] = [gate(x[p / topk]) | up(x[p / topk])]
    QmvOpts gi{};
    gi.x_row = nullptr;
    gi.x_div = (int)topk;
    gi.ldx = (int)d;
    gi.w_sel = ids;
    gi.n_experts = (int)e;
    gi.expert_bytes = gate_bytes;
    gi.w2 = static_cast<const uint8_t*>(w_up);
    gi.n_split = (int)ffn;
    if (e <= (size_t)QMV_ROUTE_MAX_EXPERTS) {  // each workgroup routes its token from the logits
        gi.w_sel = nullptr;
        gi.route_logits = logits;
        gi.route_ids = ids;
        gi.route_w = wts;
    }
    if ((rc = run_indexed(dev, dt, static_cast<const uint8_t*>(w_gate), x, p, (int)(2 * ffn), (int)d, gu,
                          (int)(2 * ffn), gi)))
        return rc;
    // down over silu(gate) * up and the combine in one launch where it fits
    if (moe_down_combine_supported(dt, (int)topk, (int)ffn)) {
        HIP_TRY(launch_moe_down_combine(dt, static_cast<const uint8_t*>(w_down), down_bytes, (int)e, gu, ids, wts,
                                        (int)t, (int)topk, (int)ffn, (int)d, out, dev->stream, dev->num_cus));
        return FRQ_OK;
    }
    // down over silu(gate) * up, quantized inside the mat-vec
    QmvOpts di{};
    di.x_row = nullptr;
    di.x_div = 1;
    di.ldx = (int)(2 * ffn);
    di.w_sel = ids;
    di.n_experts = (int)e;
    di.expert_bytes = down_bytes;
    di.x2 = gu + ffn;
    if ((rc = run_indexed(dev, dt, static_cast<const uint8_t*>(w_down), gu, p, (int)d, (int)ffn, yd, (int)d, di)))
        return rc;
    HIP_TRY(launch_moe_combine(yd, ids, wts, nullptr, (int)t, (int)topk, (int)d, out, dev->stream));
    return FRQ_OK;
}

// ---- decode-step fusions ----

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int frq_qmatmul_fused(frq_device* dev, int dt, size_t m, size_t n, size_t k, const void* w, const float* x, size_t ldx,
                      const float* x2, const float* gain, float eps, int accumulate, float* y, size_t ldy) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!is_weight_type(dt)) return fail(FRQ_UNSUPPORTED, "qmatmul_fused: dtype %d", dt);
    if (k == 0 || k % block_elems(dt))
        return fail(FRQ_INVALID, "qmatmul_fused: k=%zu must be a positive multiple of %zu", k, block_elems(dt));
    if (m > 65535 || n > (size_t)0x7fffffff) return fail(FRQ_UNSUPPORTED, "qmatmul_fused: m=%zu n=%zu", m, n);
    if (m == 0 || n == 0) return FRQ_OK;
    if (!w || !x || !y) return fail(FRQ_INVALID, "qmatmul_fused: null buffer");
    if (m > 1 && (ldx < k || ldy < n)) return fail(FRQ_INVALID, "qmatmul_fused: ldx=%zu < k or ldy=%zu < n", ldx, ldy);
    if (ldx > (size_t)0x7fffffff || ldy > (size_t)0x7fffffff) return fail(FRQ_UNSUPPORTED, "qmatmul_fused: strides");
    if (x2 && gain) return fail(FRQ_INVALID, "qmatmul_fused: rms_gain and x2 are exclusive");
    if (!aligned16(x) || (x2 && !aligned16(x2)) || (gain && !aligned16(gain)) || ldx % 4)
        return fail(FRQ_MISALIGNED, "qmatmul_fused: x, x2, gain must be 16-byte aligned and ldx %% 4 == 0");
    if (!aligned4(y) || !aligned4(w)) return fail(FRQ_MISALIGNED, "qmatmul_fused: w / y not 4-byte aligned");
    const ActSrc src{x, (int)ldx, x2, gain, eps};
    FusedBatch fb;
    if (fused_batch_plan(dev, dt, w, src, m, n, k, &fb)) {  // several rows: quantize once, one weight pass
        rc = ensure_ws(dev, fb.abytes + fb.plan.part_elems * sizeof(float));
        if (rc) return rc;
        const ActView act = act_view(dev->ws, GGML_Q8K, m, k);
        HIP_TRY(launch_quantize_q8k_src(src, (int)m, (int)k, act, dev->stream));
        HIP_TRY(launch_fused_batch(dev, fb, dt, w, act, m, n, k, y, ldy, accumulate ? OUT_ACC : 0));
        return FRQ_OK;
    }
    if (k > qmv_kmax(dt)) return fail(FRQ_UNSUPPORTED, "qmatmul_fused: k=%zu exceeds %zu", k, qmv_kmax(dt));
    QmvOpts o{};
    o.ldx = (int)ldx;
    o.x2 = x2;
    o.rms_gain = gain;
    o.rms_eps = eps;
    o.accumulate = accumulate ? 1 : 0;
    HIP_TRY(launch_qmv_fused(dt, static_cast<const uint8_t*>(w), x, y, (int)m, (int)n, (int)k, (int)ldy, o,
                             dev->stream, dev->num_cus));
    return FRQ_OK;
}

int frq_qmatmul_fused_pair(frq_device* dev, size_t m, size_t k, const float* x, size_t ldx, const float* gain,
                           float eps, int dt1, size_t n1, const void* w1, float* y1, int dt2, size_t n2, const void* w2,
                           float* y2) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!qmv_pair_supported(dt1, dt2, (int)(k > 0x7fffffff ? 0 : k)) || k == 0)
        return fail(FRQ_UNSUPPORTED, "qmatmul_fused_pair: dtypes %d/%d with k=%zu", dt1, dt2, k);
    if (m > 65535 || n1 > (size_t)0x7fffffff || n2 > (size_t)0x7fffffff)
        return fail(FRQ_UNSUPPORTED, "qmatmul_fused_pair: m=%zu n1=%zu n2=%zu", m, n1, n2);
    if (m == 0 || n1 == 0 || n2 == 0) return FRQ_OK;
    if (!x || !w1 || !w2 || !y1 || !y2) return fail(FRQ_INVALID, "qmatmul_fused_pair: null buffer");
    if ((m > 1 && ldx < k) || ldx > (size_t)0x7fffffff) return fail(FRQ_INVALID, "qmatmul_fused_pair: ldx=%zu", ldx);
    if (!aligned16(x) || (gain && !aligned16(gain)) || ldx % 4)
        return fail(FRQ_MISALIGNED, "qmatmul_fused_pair: x and gain must be 16-byte aligned and ldx %% 4 == 0");
    if (!aligned4(w1) || !aligned4(w2) || !aligned4(y1) || !aligned4(y2))
        return fail(FRQ_MISALIGNED, "qmatmul_fused_pair: weights / outputs not 4-byte aligned");
    const ActSrc src{x, (int)ldx, nullptr, gain, eps};
    FusedBatch fb1, fb2;
    if (fused_batch_plan(dev, dt1, w1, src, m, n1, k, &fb1) && fused_batch_plan(dev, dt2, w2, src, m, n2, k, &fb2)) {
        // several rows: the normalized rows quantized once for both matrices
        const size_t parts = fb1.plan.part_elems > fb2.plan.part_elems ? fb1.plan.part_elems : fb2.plan.part_elems;
        rc = ensure_ws(dev, fb1.abytes + parts * sizeof(float));
        if (rc) return rc;
        const ActView act = act_view(dev->ws, GGML_Q8K, m, k);
        HIP_TRY(launch_quantize_q8k_src(src, (int)m, (int)k, act, dev->stream));
        HIP_TRY(launch_fused_batch(dev, fb1, dt1, w1, act, m, n1, k, y1, n1, 0));
        HIP_TRY(launch_fused_batch(dev, fb2, dt2, w2, act, m, n2, k, y2, n2, 0));
        return FRQ_OK;
    }
    QmvOpts o{};
    o.ldx = (int)ldx;
    o.rms_gain = gain;
    o.rms_eps = eps;
    HIP_TRY(launch_qmv_pair(dt1, static_cast<const uint8_t*>(w1), y1, (int)n1, dt2, static_cast<const uint8_t*>(w2), y2,
                            (int)n2, x, (int)m, (int)k, o, dev->stream, dev->num_cus));
    return FRQ_OK;
}

size_t frq_attention_decode_workspace(size_t n_heads, size_t max_ctx) {
    if (n_heads == 0 || n_heads > 65535 || max_ctx == 0 || max_ctx > (size_t)0x7fffffff / (n_heads * ATTN_HEAD_DIM))
        return 0;
    return attn_decode_work_bytes((int)n_heads, (int)max_ctx);
}

int frq_attention_decode(frq_device* dev, size_t n_heads, size_t head_dim, size_t max_ctx, const float* qk,
                         const float* v, const float* rcos, const float* rsin, uint16_t* kc, uint16_t* vc,
                         const int32_t* pos, float scale, void* work, size_t work_bytes, float* out) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (head_dim != (size_t)ATTN_HEAD_DIM)
        return fail(FRQ_UNSUPPORTED, "attention_decode: head_dim=%zu (supported: %d)", head_dim, ATTN_HEAD_DIM);
    const size_t need = frq_attention_decode_workspace(n_heads, max_ctx);
    if (need == 0) return fail(FRQ_INVALID, "attention_decode: n_heads=%zu max_ctx=%zu", n_heads, max_ctx);
    if (!qk || !v || !rcos || !rsin || !kc || !vc || !pos || !work || !out)
        return fail(FRQ_INVALID, "attention_decode: null buffer");
    if (work_bytes < need) return fail(FRQ_WORKSPACE, "attention_decode: workspace %zu < %zu bytes", work_bytes, need);
    if (!aligned16(kc) || !aligned16(vc) || !aligned4(work))
        return fail(FRQ_MISALIGNED, "attention_decode: caches must be 16-byte aligned, work 4-byte aligned");
    HIP_TRY(launch_attn_decode(qk, v, rcos, rsin, kc, vc, (int)n_heads, (int)max_ctx, pos, scale,
                               static_cast<float*>(work), out, dev->stream));
    return FRQ_OK;
}

int frq_qmatmul_fused_glu(frq_device* dev, int dt, size_t m, size_t n, size_t k, const void* w_gate, const void* w_up,
                          const float* x, size_t ldx, const float* gain, float eps, float* y, size_t ldy) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!is_weight_type(dt)) return fail(FRQ_UNSUPPORTED, "qmatmul_fused_glu: dtype %d", dt);
    if (k == 0 || k % block_elems(dt))
        return fail(FRQ_INVALID, "qmatmul_fused_glu: k=%zu must be a positive multiple of %zu", k, block_elems(dt));
    if (k > qmv_kmax(dt)) return fail(FRQ_UNSUPPORTED, "qmatmul_fused_glu: k=%zu exceeds %zu", k, qmv_kmax(dt));
    if (m > 65535 || n > (size_t)0x7fffffff) return fail(FRQ_UNSUPPORTED, "qmatmul_fused_glu: m=%zu n=%zu", m, n);
    if (m == 0 || n == 0) return FRQ_OK;
    if (!w_gate || !w_up || !x || !y) return fail(FRQ_INVALID, "qmatmul_fused_glu: null buffer");
    if (m > 1 && (ldx < k || ldy < n))
        return fail(FRQ_INVALID, "qmatmul_fused_glu: ldx=%zu < k or ldy=%zu < n", ldx, ldy);
    if (ldx > (size_t)0x7fffffff || ldy > (size_t)0x7fffffff) return fail(FRQ_UNSUPPORTED, "qmatmul_fused_glu: strides");
    if (!aligned16(x) || (gain && !aligned16(gain)) || ldx % 4)
        return fail(FRQ_MISALIGNED, "qmatmul_fused_glu: x and gain must be 16-byte aligned and ldx %% 4 == 0");
    if (!aligned4(y) || !aligned4(w_gate) || !aligned4(w_up))
        return fail(FRQ_MISALIGNED, "qmatmul_fused_glu: weights / y not 4-byte aligned");
    QmvOpts o{};
    o.ldx = (int)ldx;
    o.rms_gain = gain;
    o.rms_eps = eps;
    HIP_TRY(launch_qmv_glu(dt, static_cast<const uint8_t*>(w_gate), static_cast<const uint8_t*>(w_up), x, y, (int)m,
                           (int)n, (int)k, (int)ldy, o, dev->stream, dev->num_cus));
    return FRQ_OK;
}

int frq_attention_decode_oproj(frq_device* dev, size_t n_heads, size_t head_dim, size_t max_ctx, const float* qk,
                               const float* v, const float* rcos, const float* rsin, uint16_t* kc, uint16_t* vc,
                               const int32_t* pos, float scale, void* work, size_t work_bytes, int o_dtype,
                               const void* w_o, size_t n_out, float* y) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (head_dim != (size_t)ATTN_HEAD_DIM)
        return fail(FRQ_UNSUPPORTED, "attention_decode_oproj: head_dim=%zu (supported: %d)", head_dim, ATTN_HEAD_DIM);
    const size_t need = frq_attention_decode_workspace(n_heads, max_ctx);
    if (need == 0) return fail(FRQ_INVALID, "attention_decode_oproj: n_heads=%zu max_ctx=%zu", n_heads, max_ctx);
    if (!is_weight_type(o_dtype)) return fail(FRQ_UNSUPPORTED, "attention_decode_oproj: o dtype %d", o_dtype);
    const size_t k = n_heads * head_dim;
    if (k % QK_K || k > qmv_kmax(o_dtype))
        return fail(FRQ_UNSUPPORTED, "attention_decode_oproj: n_heads * head_dim = %zu (needs a multiple of %d, <= %zu)",
                    k, QK_K, qmv_kmax(o_dtype));
    if (n_out == 0 || n_out > (size_t)0x7fffffff) return fail(FRQ_INVALID, "attention_decode_oproj: n_out=%zu", n_out);
    if (!qk || !v || !rcos || !rsin || !kc || !vc || !pos || !work || !w_o || !y)
        return fail(FRQ_INVALID, "attention_decode_oproj: null buffer");
    if (work_bytes < need)
        return fail(FRQ_WORKSPACE, "attention_decode_oproj: workspace %zu < %zu bytes", work_bytes, need);
    if (!aligned16(kc) || !aligned16(vc) || !aligned16(work) || !aligned4(w_o) || !aligned4(y))
        return fail(FRQ_MISALIGNED,
                    "attention_decode_oproj: caches and work must be 16-byte aligned, w_o and y 4-byte aligned");
    float* part = static_cast<float*>(work);
    const int ns = attn_decode_splits((int)n_heads, (int)max_ctx);
    QmvOpts o{};
    o.accumulate = 1;
    if (ns <= ATTN_MERGE_CHUNK) {  // the merge inside the mat-vec: two launches
        HIP_TRY(launch_attn_split(qk, v, rcos, rsin, kc, vc, (int)n_heads, (int)max_ctx, pos, scale, part,
                                  dev->stream));
        o.attn_nsplit = ns;
        o.attn_max_ctx = (int)max_ctx;
        o.attn_pos = pos;
        HIP_TRY(launch_qmv_attn(o_dtype, static_cast<const uint8_t*>(w_o), part, y, (int)n_out, (int)k, o,
                                dev->stream, dev->num_cus));
    } else {  // more splits than one merge step holds: the merge kernel into the workspace's tail
        float* att = part + (size_t)n_heads * ns * ATTN_PSTRIDE;
        HIP_TRY(launch_attn_decode(qk, v, rcos, rsin, kc, vc, (int)n_heads, (int)max_ctx, pos, scale, part, att,
                                   dev->stream));
        o.ldx = (int)k;
        HIP_TRY(launch_qmv_fused(o_dtype, static_cast<const uint8_t*>(w_o), att, y, 1, (int)n_out, (int)k,
                                 (int)n_out, o, dev->stream, dev->num_cus));
    }
    return FRQ_OK;
}

// ---- prefill row kernels ----

int frq_rms_norm_rows(frq_device* dev, size_t m, size_t k, const float* x, size_t ldx, const float* gain, float eps,
                      float* y, size_t ldy) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (m > 0x7fffffff || k == 0 || k > 0x7fffffff || ldx < k || ldy < k || ldx > 0x7fffffff || ldy > 0x7fffffff)
        return fail(FRQ_INVALID, "rms_norm_rows: m=%zu k=%zu ldx=%zu ldy=%zu", m, k, ldx, ldy);
    if (m == 0) return FRQ_OK;
    if (!x || !gain || !y) return fail(FRQ_INVALID, "rms_norm_rows: null buffer");
    HIP_TRY(launch_rms_norm_rows(x, (int)ldx, gain, eps, (int)m, (int)k, y, (int)ldy, dev->stream));
    return FRQ_OK;
}

int frq_rope_append_rows(frq_device* dev, size_t m, size_t n_heads, size_t head_dim, size_t max_ctx, float* qk,
                         size_t ldqk, const float* v, size_t ldv, const float* rcos, const float* rsin, size_t pos0,
                         uint16_t* kc, uint16_t* vc) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (head_dim != (size_t)ATTN_HEAD_DIM)
        return fail(FRQ_UNSUPPORTED, "rope_append_rows: head_dim=%zu (supported: %d)", head_dim, ATTN_HEAD_DIM);
    if (n_heads == 0 || n_heads > 65535 || max_ctx == 0 || max_ctx > (size_t)0x7fffffff / (n_heads * head_dim) ||
        pos0 > max_ctx || m > max_ctx - pos0)
        return fail(FRQ_INVALID, "rope_append_rows: m=%zu pos0=%zu n_heads=%zu max_ctx=%zu", m, pos0, n_heads,
                    max_ctx);
    if (ldqk < 2 * n_heads * head_dim || ldv < n_heads * head_dim || ldqk > 0x7fffffff || ldv > 0x7fffffff)
        return fail(FRQ_INVALID, "rope_append_rows: ldqk=%zu ldv=%zu", ldqk, ldv);
    if (m == 0) return FRQ_OK;
    if (m > 65535) return fail(FRQ_UNSUPPORTED, "rope_append_rows: m=%zu > 65535", m);
    if (!qk || !v || !rcos || !rsin || !kc || !vc) return fail(FRQ_INVALID, "rope_append_rows: null buffer");
    HIP_TRY(launch_rope_append_rows(qk, (int)ldqk, v, (int)ldv, rcos, rsin, (int)m, (int)n_heads, (int)pos0,
                                    (int)max_ctx, kc, vc, dev->stream));
    return FRQ_OK;
}

int frq_attention_prefill(frq_device* dev, size_t m, size_t n_heads, size_t head_dim, size_t max_ctx, const float* q,
                          size_t ldq, const uint16_t* kc, const uint16_t* vc, size_t pos0, float scale, float* out,
                          size_t ldo) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (head_dim != (size_t)ATTN_HEAD_DIM)
        return fail(FRQ_UNSUPPORTED, "attention_prefill: head_dim=%zu (supported: %d)", head_dim, ATTN_HEAD_DIM);
    if (n_heads == 0 || n_heads > 65535 || max_ctx == 0 || max_ctx > (size_t)0x7fffffff / (n_heads * head_dim) ||
        pos0 > max_ctx || m > max_ctx - pos0)
        return fail(FRQ_INVALID, "attention_prefill: m=%zu pos0=%zu n_heads=%zu max_ctx=%zu", m, pos0, n_heads,
                    max_ctx);
    if (ldq < n_heads * head_dim || ldo < n_heads * head_dim || ldq > 0x7fffffff || ldo > 0x7fffffff)
        return fail(FRQ_INVALID, "attention_prefill: ldq=%zu ldo=%zu", ldq, ldo);
    if (m == 0) return FRQ_OK;
    if (!q || !kc || !vc || !out) return fail(FRQ_INVALID, "attention_prefill: null buffer");
    if (!aligned16(kc) || !aligned16(vc)) return fail(FRQ_MISALIGNED, "attention_prefill: caches not 16-byte aligned");
    HIP_TRY(launch_attention_prefill(q, (int)ldq, kc, vc, (int)pos0, (int)m, (int)n_heads, (int)max_ctx, scale, out,
                                     (int)ldo, dev->stream));
    return FRQ_OK;
}

int frq_swiglu_rows(frq_device* dev, size_t m, size_t f, const float* gu, size_t ldgu, float* h, size_t ldh) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (m > 65535 || f == 0 || f > 0x7fffffff || ldgu < 2 * f || ldh < f || ldgu > 0x7fffffff || ldh > 0x7fffffff)
        return fail(FRQ_INVALID, "swiglu_rows: m=%zu f=%zu ldgu=%zu ldh=%zu", m, f, ldgu, ldh);
    if (m == 0) return FRQ_OK;
    if (!gu || !h) return fail(FRQ_INVALID, "swiglu_rows: null buffer");
    HIP_TRY(launch_swiglu_rows(gu, (int)ldgu, (int)m, (int)f, h, (int)ldh, dev->stream));
    return FRQ_OK;
}

int frq_add(frq_device* dev, size_t n, const float* x, float* y) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (n == 0) return FRQ_OK;
    if (!x || !y) return fail(FRQ_INVALID, "add: null buffer");
    if (n / 256 >= 0x7fffffff) return fail(FRQ_UNSUPPORTED, "add: n=%zu", n);
    HIP_TRY(launch_add_rows(x, y, n, dev->stream));
    return FRQ_OK;
}

int frq_gather_rows(frq_device* dev, const float* table, size_t rows, size_t dim, const int32_t* ids, size_t m,
                    float* out) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (rows == 0 || rows > 0x7fffffff || dim == 0 || dim > 0x7fffffff || m > 65535)
        return fail(FRQ_INVALID, "gather_rows: rows=%zu dim=%zu m=%zu", rows, dim, m);
    if (m == 0) return FRQ_OK;
    if (!table || !ids || !out) return fail(FRQ_INVALID, "gather_rows: null buffer");
    HIP_TRY(launch_gather_rows(table, (int)rows, (int)dim, ids, (int)m, out, dev->stream));
    return FRQ_OK;
}

int frq_argmax_embed(frq_device* dev, const float* logits, size_t vocab, const float* table, size_t dim, int32_t* tokens,
                     size_t tokens_cap, const int32_t* prompt_len, int32_t* pos, float* x) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (vocab == 0 || vocab > (size_t)0x7fffffff || dim == 0 || dim % 4 || tokens_cap > (size_t)0x7fffffff)
        return fail(FRQ_INVALID, "argmax_embed: vocab=%zu dim=%zu", vocab, dim);
    if (!logits || !table || !tokens || !prompt_len || !pos || !x) return fail(FRQ_INVALID, "argmax_embed: null buffer");
    if (!aligned16(table) || !aligned16(x)) return fail(FRQ_MISALIGNED, "argmax_embed: table / x not 16-byte aligned");
    HIP_TRY(launch_argmax_embed(logits, (int)vocab, table, (int)dim, tokens, (int)tokens_cap, prompt_len, pos, x,
                                dev->stream));
    return FRQ_OK;
}

int frq_fill_random_bits(frq_device* dev, uint32_t* y, size_t n, uint64_t start, uint64_t seed, uint32_t base,
                         uint32_t stream) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (n && !y) return fail(FRQ_INVALID, "null output");
    HIP_TRY(launch_random_bits(y, n, start, seed, base, stream, dev->stream));
    return FRQ_OK;
}

int frq_fill_normal(frq_device* dev, float* y, size_t n, uint64_t seed, uint32_t stream, float mean, float stdv) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (n && !y) return fail(FRQ_INVALID, "null output");
    if (!aligned4(y)) return fail(FRQ_MISALIGNED, "fill_normal: output not 4-byte aligned");
    HIP_TRY(launch_normal(y, n, seed, stream, mean, stdv, dev->stream));
    return FRQ_OK;
}

int frq_probe_read(frq_device* dev, const void* src, size_t bytes, int wg_per_cu, int unroll, int nontemporal,
                   uint32_t* sink) {
    DevGuard guard(dev);
    int rc = use_device(dev);
    if (rc) return rc;
    if (!src || !sink) return fail(FRQ_INVALID, "probe_read: null buffer");
    if (!aligned16(src) || bytes % 16 || !bytes) return fail(FRQ_MISALIGNED, "probe_read: 16-byte aligned, whole 16-byte words");
    if (wg_per_cu < 1 || wg_per_cu > 32 || (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8))
        return fail(FRQ_INVALID, "probe_read: wg_per_cu %d (1..32), unroll %d (1, 2, 4, 8)", wg_per_cu, unroll);
    HIP_TRY(launch_probe_read(src, bytes, wg_per_cu * dev->num_cus, unroll, nontemporal, sink, dev->stream));
    return FRQ_OK;
}

// ---- GGUF files ----

namespace {
const frq::gguf::Value* gv(const frq_gguf_value* v) { return reinterpret_cast<const frq::gguf::Value*>(v); }
const frq_gguf_value* gh(const frq::gguf::Value* v) { return reinterpret_cast<const frq_gguf_value*>(v); }
}  // namespace

int frq_gguf_open(const char* path, frq_gguf** out) {
    if (!path || !out) return fail(FRQ_INVALID, "gguf_open: null argument");
    *out = nullptr;
    std::string err;
    std::unique_ptr<frq::gguf::File> f = frq::gguf::open(path, err);
    if (!f) return fail(FRQ_INVALID, "%s", err.c_str());
    *out = new frq_gguf{std::move(f)};
    return FRQ_OK;
}

int frq_gguf_close(frq_gguf* g) {
    delete g;
    return FRQ_OK;
}

int frq_gguf_version(const frq_gguf* g) { return g ? g->f->version : -1; }
uint64_t frq_gguf_tensor_data_offset(const frq_gguf* g) { return g ? g->f->tensor_data_offset : 0; }
size_t frq_gguf_tensor_count(const frq_gguf* g) { return g ? g->f->tensors.size() : 0; }
size_t frq_gguf_meta_count(const frq_gguf* g) { return g ? g->f->metadata.size() : 0; }

int frq_gguf_tensor_info(const frq_gguf* g, size_t index, const char** name, int* ggml_dtype, size_t* n_dims,
                         uint64_t* dims, size_t dims_cap, uint64_t* offset, uint64_t* nbytes) {
    if (!g) return fail(FRQ_INVALID, "null gguf");
    if (index >= g->f->tensors.size()) return fail(FRQ_INVALID, "gguf: tensor index %zu of %zu", index, g->f->tensors.size());
    const frq::gguf::TensorInfo& t = g->f->tensors[index];
    if (name) *name = t.name.c_str();
    if (ggml_dtype) *ggml_dtype = t.ggml_dtype;
    if (n_dims) *n_dims = t.dims.size();
    if (dims) {
        if (t.dims.size() > dims_cap)
            return fail(FRQ_INVALID, "gguf: tensor %s has %zu dims, buffer holds %zu", t.name.c_str(), t.dims.size(),
                        dims_cap);
        for (size_t i = 0; i < t.dims.size(); i++) dims[i] = t.dims[i];
    }
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return FRQ_OK;
}

int frq_gguf_find_tensor(const frq_gguf* g, const char* name, size_t* index) {
    if (!g || !name || !index) return fail(FRQ_INVALID, "gguf_find_tensor: null argument");
    auto it = g->f->tensor_index.find(name);
    if (it == g->f->tensor_index.end()) return fail(FRQ_INVALID, "gguf: missing tensor \"%s\"", name);
    *index = it->second;
    return FRQ_OK;
}

int frq_gguf_tensor_data(const frq_gguf* g, size_t index, const void** host, uint64_t* nbytes) {
    if (!g || !host || !nbytes) return fail(FRQ_INVALID, "gguf_tensor_data: null argument");
    const frq::gguf::File& f = *g->f;
    if (index >= f.tensors.size()) return fail(FRQ_INVALID, "gguf: tensor index %zu of %zu", index, f.tensors.size());
    const frq::gguf::TensorInfo& t = f.tensors[index];
    const unsigned __int128 start = (unsigned __int128)f.tensor_data_offset + t.offset;
    if (start + t.nbytes > f.map_bytes)
        return fail(FRQ_INVALID, "gguf: tensor %s bytes [%llu, +%llu) lie outside the %zu-byte file", t.name.c_str(),
                    (unsigned long long)start, (unsigned long long)t.nbytes, f.map_bytes);
    *host = f.map + (size_t)start;
    *nbytes = t.nbytes;
    return FRQ_OK;
}

int frq_gguf_load_quantized(frq_device* dev, const frq_gguf* g, size_t index, frq_qstorage** out) {
    const void* host = nullptr;
    uint64_t nbytes = 0;
    int rc = frq_gguf_tensor_data(g, index, &host, &nbytes);
    if (rc) return rc;
    const int dt = g->f->tensors[index].ggml_dtype;
    if (!type_size(dt))
        return fail(FRQ_UNSUPPORTED, "gguf: tensor %s has dtype %d, not a quantized storage type",
                    g->f->tensors[index].name.c_str(), dt);
    return frq_qstorage_load(dev, dt, host, (size_t)nbytes, out);
}

int frq_gguf_meta_at(const frq_gguf* g, size_t index, const char** key, const frq_gguf_value** value) {
    if (!g) return fail(FRQ_INVALID, "null gguf");
    if (index >= g->f->metadata.size())
        return fail(FRQ_INVALID, "gguf: metadata index %zu of %zu", index, g->f->metadata.size());
    if (key) *key = g->f->metadata[index].first.c_str();
    if (value) *value = gh(&g->f->metadata[index].second);
    return FRQ_OK;
}

int frq_gguf_meta_find(const frq_gguf* g, const char* key, const frq_gguf_value** value) {
    if (!g || !key || !value) return fail(FRQ_INVALID, "gguf_meta_find: null argument");
    auto it = g->f->meta_index.find(key);
    if (it == g->f->meta_index.end()) return fail(FRQ_INVALID, "cannot find %s in metadata", key);
    *value = gh(&g->f->metadata[it->second].second);
    return FRQ_OK;
}

int frq_gguf_value_type(const frq_gguf_value* v) { return v ? gv(v)->type : -1; }

int frq_gguf_value_scalar(const frq_gguf_value* v, uint64_t* u, int64_t* i, double* f) {
    if (!v) return fail(FRQ_INVALID, "null value");
    const frq::gguf::Value& x = *gv(v);
    if (x.type == frq::gguf::VT_STRING || x.type == frq::gguf::VT_ARRAY)
        return fail(FRQ_INVALID, "gguf: value of type %d is not a scalar", x.type);
    if (u) *u = x.u;
    if (i) *i = x.i;
    if (f) *f = x.f;
    return FRQ_OK;
}

int frq_gguf_value_u64(const frq_gguf_value* v, uint64_t* out) {
    if (!v || !out) return fail(FRQ_INVALID, "null argument");
    const frq::gguf::Value& x = *gv(v);
    // Value::to_u64: U64, U8 / U16 / U32 and Bool upcast (gguf.rs:262-272)
    if (x.type == frq::gguf::VT_U64 || x.type == frq::gguf::VT_U8 || x.type == frq::gguf::VT_U16 ||
        x.type == frq::gguf::VT_U32 || x.type == frq::gguf::VT_BOOL) {
        *out = x.u;
        return FRQ_OK;
    }
    return fail(FRQ_INVALID, "not a u64 or upcastable to u64 (value type %d)", x.type);
}

int frq_gguf_value_string(const frq_gguf_value* v, const char** s, size_t* len) {
    if (!v || !s || !len) return fail(FRQ_INVALID, "null argument");
    const frq::gguf::Value& x = *gv(v);
    if (x.type != frq::gguf::VT_STRING) return fail(FRQ_INVALID, "not a string (value type %d)", x.type);
    *s = x.s.c_str();
    *len = x.s.size();
    return FRQ_OK;
}

int frq_gguf_value_array(const frq_gguf_value* v, size_t* len) {
    if (!v || !len) return fail(FRQ_INVALID, "null argument");
    const frq::gguf::Value& x = *gv(v);
    if (x.type != frq::gguf::VT_ARRAY) return fail(FRQ_INVALID, "not a vec (value type %d)", x.type);
    *len = x.a.size();
    return FRQ_OK;
}

int frq_gguf_value_array_at(const frq_gguf_value* v, size_t j, const frq_gguf_value** elem) {
    size_t len = 0;
    int rc = frq_gguf_value_array(v, &len);
    if (rc) return rc;
    if (!elem) return fail(FRQ_INVALID, "null argument");
    if (j >= len) return fail(FRQ_INVALID, "gguf: array index %zu of %zu", j, len);
    *elem = gh(&gv(v)->a[j]);
    return FRQ_OK;
}

}  // extern "C"
