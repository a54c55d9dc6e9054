// om_hip.hip — the C-ABI of include/om_hip.h on the HIP runtime.
//
// Owns the device copies of each GDN layer's weights and per-sequence state
// (the engine's conv_st / rec_st, engines/qwen.c:275-276) and the grow-only
// scratch the entry points need (the om_metal ensure() precedent,
// metal/om_metal.mm:148-151).  Host-pointer calls run on a library stream
// and block until done (om_metal's waitUntilCompleted); *_dev calls only
// enqueue on the caller's stream.
#include "om_hip.h"
#include "omh_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

using namespace omh;

namespace {

constexpr int kMaxLayers = 4096;

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

#define HIP_OK(expr)                                                                      \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(OMH_ERR_DEVICE, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_),   \
                        __FILE__, __LINE__);                                              \
    } while (0)

struct DevLayer {
    bool live = false;
    omh_gdn_dims d{};
    int max_seqs = 0, conv_dim = 0, vdim = 0;
    // core weights and state (conv history as a ring, omh_internal.h)
    float *conv_w = nullptr, *A_log = nullptr, *dt_bias = nullptr, *gnorm = nullptr;
    float *conv_st = nullptr, *S = nullptr;
    int *phase = nullptr;                  // [2][max_seqs]
    int epoch = 0;                         // which phase buffer decode launches read
    float *o_raw = nullptr, *ssq = nullptr;
    int *cnt = nullptr;
    // projections: in_proj rows [qkv | z | b | a]; rows < in_nq are int8
    bool has_proj = false;
    int in_rows = 0, in_nq = 0;
    int8_t *Qin = nullptr;
    float *Sin = nullptr, *Win = nullptr;
    int out_nq = 0;
    int8_t *Qout = nullptr;
    float *Sout = nullptr, *Wout = nullptr;
    int8_t *Qtin = nullptr, *Qtout = nullptr;   // tiled copies of the int8 rows (tile_q8), or null
};

DevLayer g_L[kMaxLayers];
int g_ready = -1;
hipStream_t g_stream = nullptr;

// grow-only device scratch
struct Scratch {
    void *p = nullptr;
    size_t n = 0;
};
Scratch g_x, g_out, g_in, g_core, g_qkv, g_z, g_a, g_b, g_pre, g_xb, g_dec;


// k-split arrival counters of the projections: zeroed once at init and
// zero between launches (each tile's last arriver resets its own), shared
// by every call (calls that may overlap must come from one stream)
constexpr int kCounters = 1 << 18;
int *g_counters = nullptr;

int ensure(Scratch &s, size_t bytes) {
    if (bytes <= s.n) return OMH_OK;
    if (s.p) (void)hipFree(s.p);
    s.p = nullptr;
    s.n = 0;
    size_t want = bytes < 4096 ? 4096 : bytes;
    if (hipMalloc(&s.p, want) != hipSuccess) return fail(OMH_ERR_ALLOC, "scratch alloc of %zu bytes failed", want);
    s.n = want;
    return OMH_OK;
}

// Pinned, device-mapped host staging for the synchronous small calls (one
// decode token, a short attention step): x is copied into it on the CPU and
// sent with one asynchronous copy; the last projection writes its output
// straight into the mapped output buffer, so no device-to-host copy is
// queued.  One call of the 35B GDN layer at one token: 31.5 us against
// 47 us with pageable copies both ways (MI355X).  Grow-only.
struct Pinned {
    float *h = nullptr;         // host address
    float *d = nullptr;         // the device's address of the same memory
    size_t n = 0;               // bytes
};
Pinned g_hx, g_hout;
constexpr size_t kPinnedMaxBytes = size_t(1) << 20;   // calls above this use pageable copies

int ensure_pinned(Pinned &b, size_t bytes) {
    if (bytes <= b.n) return OMH_OK;
    if (b.h) (void)hipHostFree(b.h);
    b = Pinned{};
    void *h = nullptr, *d = nullptr;
    if (hipHostMalloc(&h, bytes, hipHostMallocMapped) != hipSuccess) return fail(OMH_ERR_ALLOC, "pinned staging of %zu bytes failed", bytes);
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
        (void)hipHostFree(h);
        return fail(OMH_ERR_ALLOC, "pinned staging: no device address");
    }
    b.h = static_cast<float *>(h);
    b.d = static_cast<float *>(d);
    b.n = bytes;
    return OMH_OK;
}

// Stage n floats of x for the device (pinned copy, then one async copy into
// g_x) and make sure the mapped output buffer holds n_out floats.  Small
// calls only (kPinnedMaxBytes), whose last projection is the register GEMV
// (up to 4 tokens): it writes each output once, 16 rows per store wave.
int stage_small(const float *x, size_t n, size_t n_out) {
    if (int rc = ensure_pinned(g_hx, n * 4)) return rc;
    if (int rc = ensure_pinned(g_hout, n_out * 4)) return rc;
    if (int rc = ensure(g_x, n * 4)) return rc;
    memcpy(g_hx.h, x, n * 4);
    HIP_OK(hipMemcpyAsync(g_x.p, g_hx.h, n * 4, hipMemcpyHostToDevice, g_stream));
    return OMH_OK;
}

template <typename T>
int upload(T **dst, size_t count, const T *src) {
    if (hipMalloc(reinterpret_cast<void **>(dst), count * sizeof(T) + 16) != hipSuccess)
        return fail(OMH_ERR_ALLOC, "alloc of %zu bytes failed", count * sizeof(T));
    if (src) HIP_OK(hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice));
    return OMH_OK;
}

// The tiled copy of O x I int8 weights the prefill-sized GEMM reads
// (tile_q8), where the shape takes one; *Qt stays null otherwise.
int upload_tiled(int8_t **Qt, const int8_t *Q, int O, int I) {
    if (!tile_q8_wanted(O, I)) return OMH_OK;
    if (hipMalloc(reinterpret_cast<void **>(Qt), tile_q8_bytes(O, I)) != hipSuccess)
        return fail(OMH_ERR_ALLOC, "alloc of %zu bytes failed", tile_q8_bytes(O, I));
    HIP_OK(tile_q8(Q, O, I, *Qt, nullptr));
    HIP_OK(hipDeviceSynchronize());
    return OMH_OK;
}

void free_layer(DevLayer &L) {
    void *ps[] = {L.conv_w, L.A_log, L.dt_bias, L.gnorm, L.conv_st, L.S, L.phase, L.o_raw, L.ssq,
                  L.cnt, L.Qin, L.Sin, L.Win, L.Qout, L.Sout, L.Wout, L.Qtin, L.Qtout};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    L = DevLayer{};
}

int check_layer(int li) {
    if (li < 0 || li >= kMaxLayers || !g_L[li].live) return fail(OMH_ERR_ARG, "layer %d not initialised", li);
    return OMH_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

LayerPtrs ptrs(const DevLayer &L) {
    LayerPtrs p;
    p.conv_w = L.conv_w; p.A_log = L.A_log; p.dt_bias = L.dt_bias; p.gnorm = L.gnorm;
    p.conv_st = L.conv_st; p.S = L.S; p.phase = L.phase;
    p.o_raw = L.o_raw; p.ssq = L.ssq; p.cnt = L.cnt;
    p.epoch = L.epoch; p.max_seqs = L.max_seqs;
    return p;
}

// Decode kernel override for tuning and tests, read per call:
// OMH_DECODE_KERNEL=paired, or =sliced with OMH_DECODE_NCS (1, 2, 4 or 8)
// column slices per value head.  Unset: chosen by launch size.
int decode_variant() {
    const char *k = getenv("OMH_DECODE_KERNEL");
    if (k && strcmp(k, "paired") == 0) return kDecodePaired;
    if (k && strcmp(k, "sliced") == 0) {
        const char *e = getenv("OMH_DECODE_NCS");
        return e ? atoi(e) : 1;
    }
    return 0;
}

// Core decode on device pointers for layers lis[0..nl), B sequences each.
// planes: or null; with one layer, where the core output also goes as the
// out_proj scratch's bf16 planes and block sums (DecodeArgs::xb)
int decode_core(int nl, const int *lis, int B, const float *qkv, int64_t ld_qkv, const float *z,
                int64_t ld_z, const float *a, const float *b, int64_t ld_ab, float *core,
                hipStream_t st, uint16_t *planes = nullptr, int b0 = 0, bool planes_i8 = false,
                int variant_req = 0, float *ssq_out = nullptr) {
    if (nl < 1 || !lis) return fail(OMH_ERR_ARG, "decode_core: nl=%d", nl);
    for (int i = 0; i < nl; i++) {
        if (int rc = check_layer(lis[i])) return rc;
        for (int j = 0; j < i; j++)
            if (lis[j] == lis[i]) return fail(OMH_ERR_ARG, "decode_core: layer %d listed twice", lis[i]);
    }
    const DevLayer &L0 = g_L[lis[0]];
    const omh_gdn_dims &d = L0.d;
    for (int i = 1; i < nl; i++) {
        const omh_gdn_dims &e = g_L[lis[i]].d;
        if (e.kh != d.kh || e.vh != d.vh || e.kd != d.kd || e.vd != d.vd || e.conv_k != d.conv_k)
            return fail(OMH_ERR_ARG, "decode_core: layers %d and %d differ in shape", lis[0], lis[i]);
    }
    for (int i = 0; i < nl; i++)
        if (B < 1 || b0 < 0 || b0 + B > g_L[lis[i]].max_seqs)
            return fail(OMH_ERR_ARG, "decode_core: sequences %d..%d outside [0, %d) for layer %d", b0, b0 + B - 1,
                        g_L[lis[i]].max_seqs, lis[i]);
    if (!decode_core_supported(d.kd, d.vd, d.vh / d.kh, d.conv_k))
        return fail(OMH_ERR_SHAPE, "decode_core: kd=%d vd=%d rep=%d K=%d unsupported", d.kd, d.vd,
                    d.vh / d.kh, d.conv_k);
    if (!qkv || !z || !a || !b || !core) return fail(OMH_ERR_ARG, "decode_core: null pointer");
    if (!aligned16(z) || !aligned16(core) || (ld_z % 4) != 0)
        return fail(OMH_ERR_ARG, "decode_core: z/core must be 16-byte aligned rows");
    const int vdim = L0.vdim;
    const int variant = variant_req ? variant_req : decode_variant();
    // one layer's large batch as launches that each fit one round of
    // resident workgroups (one B = 64 launch at the 35B shape: 52.1 us;
    // two B = 32 launches: 2 x 23.7 us)
    const int Bc = decode_seqs_per_launch(d.kd, d.vd, d.kh, d.vh, nl, B, variant);
    for (int l0 = 0; l0 < nl; l0 += kMaxDecodeLayers) {
        const int n = nl - l0 < kMaxDecodeLayers ? nl - l0 : kMaxDecodeLayers;
        for (int c0 = 0; c0 < B; c0 += Bc) {
            const int len = B - c0 < Bc ? B - c0 : Bc;
            DecodeArgs A{};
            const size_t t0 = (size_t)l0 * B + c0;     // (Bc < B only with one layer)
            A.qkv = qkv + t0 * ld_qkv;
            A.z = z + t0 * ld_z;
            A.a = a + t0 * ld_ab;
            A.b = b + t0 * ld_ab;
            A.core = core + t0 * vdim;
            A.ld_qkv = ld_qkv; A.ld_z = ld_z; A.ld_ab = ld_ab;
            A.B = len; A.nl = n; A.kh = d.kh; A.vh = d.vh; A.rep = d.vh / d.kh; A.K = d.conv_k; A.eps = d.eps;
            A.xb = nl == 1 ? planes : nullptr;
            A.xb_i8 = planes_i8;
            A.xb_T = B;
            A.xb_t0 = c0;
            A.b0 = b0 + c0;
            A.ssq_out = ssq_out;
            for (int i = 0; i < n; i++) A.L[i] = ptrs(g_L[lis[l0 + i]]);
            HIP_OK(launch_decode_core(A, d.kd, d.vd, variant, st));
            for (int i = 0; i < n; i++) g_L[lis[l0 + i]].epoch ^= 1;
        }
    }
    return OMH_OK;
}

// Scratch of one whole-layer decode call of B sequences, as byte offsets in
// one region: the in_proj rows [B][in_rows] and core rows [B][vdim] (fp32),
// the core slices' sums of squares [B][vh][slices] (deferred norm), then,
// for int8 rows with B > 4, the projections' bf16 planes, block sums,
// k-split partial tiles and arrival counters (proj_xb_bytes).
struct DecodeScratch {
    size_t in = 0, core = 0, ssq = 0, xb = 0, xb_n = 0, total = 0;
};

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

DecodeScratch decode_scratch(const DevLayer &L, int B) {
    DecodeScratch s;
    s.in = 0;
    s.core = align256((size_t)B * L.in_rows * sizeof(float));
    s.ssq = s.core + align256((size_t)B * L.vdim * sizeof(float));
    s.xb = s.ssq + align256((size_t)B * L.d.vh * kMaxSlices * sizeof(float));
    if (B > 4 && (L.in_nq > 0 || L.out_nq > 0))
        s.xb_n = std::max(proj_xb_bytes(B, L.d.hidden, L.in_nq), proj_xb_bytes(B, L.vdim, L.out_nq));
    s.total = s.xb + align256(s.xb_n);
    return s;
}

int decode_full_args(int li, int B, const float *x, float *out) {
    if (int rc = check_layer(li)) return rc;
    const DevLayer &L = g_L[li];
    if (!L.has_proj) return fail(OMH_ERR_ARG, "layer %d was initialised without projections", li);
    if (B < 1 || B > L.max_seqs) return fail(OMH_ERR_ARG, "decode: B=%d outside [1, %d]", B, L.max_seqs);
    if (!x || !out || !aligned16(x) || !aligned16(out)) return fail(OMH_ERR_ARG, "decode: x/out must be 16-byte aligned");
    return OMH_OK;
}

// The whole layer for B sequences with its scratch at `scr` (laid out as
// decode_scratch(L, B) says) and ncnt always-zero k-split counters at cnt;
// allocates nothing.
int decode_full_on(int li, int B, const float *x, float *out, hipStream_t st, char *scr, int *cnt, int ncnt) {
    DevLayer &L = g_L[li];
    const int D = L.d.hidden;
    const DecodeScratch ds = decode_scratch(L, B);
    float *in = reinterpret_cast<float *>(scr + ds.in), *core = reinterpret_cast<float *>(scr + ds.core);
    uint16_t *xb = ds.xb_n ? reinterpret_cast<uint16_t *>(scr + ds.xb) : nullptr;
    ProjArgs p{};
    p.counters = cnt; p.ncounters = ncnt;
    p.x = x; p.ldx = D; p.y = in; p.ldy = L.in_rows; p.xb = xb; p.xb_n = ds.xb_n;
    p.Q = L.Qin; p.Qt = L.Qtin; p.scale = L.Sin; p.W = L.Win; p.T = B; p.I = D; p.O = L.in_rows; p.n_q = L.in_nq;
    HIP_OK(launch_proj(p, st));
    const int vh = L.d.vh;
    const float *zz = in + L.conv_dim, *bb = zz + L.vdim, *aa = bb + vh;
    // the core writes out_proj's bf16 planes itself, saving the split launch;
    // at up to 4 tokens with int8 out_proj rows (the GEMV) the core runs as
    // column slices that leave the gated norm's 1 / rms to the GEMV instead
    const bool i8 = proj_x_int8_planes(B, L.vdim, L.out_nq);
    uint16_t *planes = xb && L.out_nq > 0 && decode_planes_supported(L.d.vd, decode_variant(), i8) ? xb : nullptr;
    const int defer = B <= 4 && L.out_nq == D && !planes && decode_variant() == 0 && L.d.kh * B < 256
                          ? decode_deferred_slices(L.d.kd, L.d.vd) : 0;
    float *ssq = defer ? reinterpret_cast<float *>(scr + ds.ssq) : nullptr;
    if (int rc = decode_core(1, &li, B, in, L.in_rows, zz, L.in_rows, aa, bb, L.in_rows, core, st, planes, 0, i8,
                             defer, ssq))
        return rc;
    ProjArgs q{};
    q.counters = cnt; q.ncounters = ncnt;
    q.x = core; q.ldx = L.vdim; q.y = out; q.ldy = D; q.xb = xb; q.xb_n = ds.xb_n; q.x_split = planes != nullptr;
    q.Q = L.Qout; q.Qt = L.Qtout; q.scale = L.Sout; q.W = L.Wout; q.T = B; q.I = L.vdim; q.O = D; q.n_q = L.out_nq;
    if (defer) {
        q.gssq = ssq; q.gvd = L.d.vd; q.geps = L.d.eps;
    }
    HIP_OK(launch_proj(q, st));
    return OMH_OK;
}

int decode_full(int li, int B, const float *x, float *out, hipStream_t st) {
    if (int rc = decode_full_args(li, B, x, out)) return rc;
    if (int rc = ensure(g_dec, decode_scratch(g_L[li], B).total)) return rc;
    return decode_full_on(li, B, x, out, st, static_cast<char *>(g_dec.p), g_counters, kCounters);
}

// ---- the allocation-free decode entry point ----
//
// Its scratch is this file-scope array: one copy per GPU, held until the
// process ends.  Host code never passes the array's name to a kernel or a
// copy (on the host it is only a stand-in for the symbol): it uses the device
// address hipGetSymbolAddress returns, fetched once per device.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
// its first 64 KiB: the projections' k-split counters (zero at load, and
// zero again after every launch: each tile's last arriver resets its own)
constexpr size_t kNoAllocCounterBytes = size_t(64) << 10;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
char *g_scratch_dev[kMaxDevices];

int noalloc_scratch(char **out) {
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(OMH_ERR_DEVICE, "device %d beyond the library's table", dev);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch_dev[dev] = static_cast<char *>(p);
    }
    *out = g_scratch_dev[dev];
    return OMH_OK;
}

// Chunked prefill of T tokens of sequence seq on device pointers.
int prefill_core(int li, int seq, int T, const float *qkv, int64_t ld_qkv, const float *z, int64_t ld_z,
                 const float *a, const float *b, int64_t ld_ab, float *core, hipStream_t st) {
    if (int rc = check_layer(li)) return rc;
    DevLayer &L = g_L[li];
    const omh_gdn_dims &d = L.d;
    if (seq < 0 || seq >= L.max_seqs) return fail(OMH_ERR_ARG, "prefill: seq %d outside [0, %d)", seq, L.max_seqs);
    if (T < 0) return fail(OMH_ERR_ARG, "prefill: T=%d", T);
    if (T == 0) return OMH_OK;
    if (!prefill_supported(d.kd, d.vd, d.vh / d.kh, d.conv_k))
        return fail(OMH_ERR_SHAPE, "prefill: kd=%d vd=%d rep=%d K=%d unsupported", d.kd, d.vd, d.vh / d.kh, d.conv_k);
    if (!qkv || !z || !a || !b || !core) return fail(OMH_ERR_ARG, "prefill: null pointer");
    if (!aligned16(z) || !aligned16(core) || (ld_z % 4) != 0)
        return fail(OMH_ERR_ARG, "prefill: z/core must be 16-byte aligned rows");
    const int D = d.kd;
    PrefillArgs A{};
    A.qkv = qkv; A.ld_qkv = ld_qkv; A.z = z; A.ld_z = ld_z; A.a = a; A.b = b; A.ld_ab = ld_ab; A.core = core;
    A.L = ptrs(L);
    A.seq = seq; A.T = T; A.nc = (T + kChunk - 1) / kChunk; A.Tp = A.nc * kChunk;
    A.kh = d.kh; A.vh = d.vh; A.K = d.conv_k; A.eps = d.eps;
    if (int rc = ensure(g_pre, prefill_scratch_bytes(D, d.kh, d.vh, T))) return rc;
    prefill_bind_scratch(A, D, g_pre.p);
    HIP_OK(launch_prefill_core(A, D, st));
    L.epoch ^= 1;                      // the conv commit wrote the other phase buffer
    return OMH_OK;
}

int prefill_full(int li, int seq, int T, const float *x, float *out, hipStream_t st) {
    if (int rc = check_layer(li)) return rc;
    DevLayer &L = g_L[li];
    if (!L.has_proj) return fail(OMH_ERR_ARG, "layer %d was initialised without projections", li);
    if (T < 0) return fail(OMH_ERR_ARG, "prefill: T=%d", T);
    if (T == 0) return OMH_OK;
    if (!x || !out || !aligned16(x) || !aligned16(out)) return fail(OMH_ERR_ARG, "prefill: x/out must be 16-byte aligned");
    const int D = L.d.hidden;
    if (int rc = ensure(g_in, (size_t)T * L.in_rows * sizeof(float))) return rc;
    if (int rc = ensure(g_core, (size_t)T * L.vdim * sizeof(float))) return rc;
    uint16_t *xb = nullptr;
    if (T > 4 && (L.in_nq > 0 || L.out_nq > 0)) {
        const size_t xbn = std::max(proj_xb_bytes(T, D, L.in_nq), proj_xb_bytes(T, L.vdim, L.out_nq));
        if (int rc = ensure(g_xb, xbn)) return rc;
        xb = static_cast<uint16_t *>(g_xb.p);
    }
    float *in = static_cast<float *>(g_in.p), *core = static_cast<float *>(g_core.p);
    ProjArgs p{};
    p.counters = g_counters; p.ncounters = kCounters;
    p.x = x; p.ldx = D; p.y = in; p.ldy = L.in_rows; p.xb = xb; p.xb_n = xb ? g_xb.n : 0;
    p.Q = L.Qin; p.Qt = L.Qtin; p.scale = L.Sin; p.W = L.Win; p.T = T; p.I = D; p.O = L.in_rows; p.n_q = L.in_nq;
    HIP_OK(launch_proj(p, st));
    const int vh = L.d.vh;
    const float *zz = in + L.conv_dim, *bb = zz + L.vdim, *aa = bb + vh;
    if (int rc = prefill_core(li, seq, T, in, L.in_rows, zz, L.in_rows, aa, bb, L.in_rows, core, st)) return rc;
    ProjArgs q{};
    q.counters = g_counters; q.ncounters = kCounters;
    q.x = core; q.ldx = L.vdim; q.y = out; q.ldy = D; q.xb = xb; q.xb_n = xb ? g_xb.n : 0;
    q.Q = L.Qout; q.Qt = L.Qtout; q.scale = L.Sout; q.W = L.Wout; q.T = T; q.I = L.vdim; q.O = D; q.n_q = L.out_nq;
    HIP_OK(launch_proj(q, st));
    return OMH_OK;
}

// ---- gated full-attention layers (engines/qwen.c:366-425) ----
struct AttnLayer {
    bool live = false;
    omh_attn_dims d{};
    int max_seqs = 0, rows = 0, nq = 0, qdim = 0;   // projection rows [H x (q|gate), KV x k, KV x v]; int8 rows; H*hd
    int8_t *Qin = nullptr;
    float *Sin = nullptr, *Win = nullptr;
    int out_nq = 0;
    int8_t *Qout = nullptr;
    float *Sout = nullptr, *Wout = nullptr;
    int8_t *Qtin = nullptr, *Qtout = nullptr;   // tiled copies of the int8 rows (tile_q8), or null
    float *qn = nullptr, *kn = nullptr, *inv = nullptr;
    float *Kc = nullptr, *Vc = nullptr;
};
AttnLayer g_A[kMaxLayers];
Scratch g_arow, g_aqb, g_actx, g_apo, g_apml, g_aimg;

void free_attn(AttnLayer &A) {
    void *ps[] = {A.Qin, A.Sin, A.Win, A.Qout, A.Sout, A.Wout, A.Qtin, A.Qtout, A.qn, A.kn, A.inv, A.Kc, A.Vc};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    A = AttnLayer{};
}

int check_attn(int li) {
    if (li < 0 || li >= kMaxLayers || !g_A[li].live) return fail(OMH_ERR_ARG, "attention layer %d not initialised", li);
    return OMH_OK;
}

int attn_forward(int li, int seq, int pos, int T, const float *x, float *out, hipStream_t st) {
    if (int rc = check_attn(li)) return rc;
    const AttnLayer &A = g_A[li];
    const omh_attn_dims &d = A.d;
    if (seq < 0 || seq >= A.max_seqs) return fail(OMH_ERR_ARG, "attn: seq %d outside [0, %d)", seq, A.max_seqs);
    if (T < 0 || pos < 0 || (long)pos + T > d.max_t)
        return fail(OMH_ERR_ARG, "attn: positions %d..%d outside the cache of %d", pos, pos + T - 1, d.max_t);
    if (T == 0) return OMH_OK;
    if (!x || !out || !aligned16(x) || !aligned16(out)) return fail(OMH_ERR_ARG, "attn: x/out must be 16-byte aligned");
    const int D = d.hidden, hd = d.head_dim, H = d.n_heads;
    int ns = 0, kps = 0;
    attn_plan(pos, T, d.n_kv, ns, kps);
    const size_t nth = (size_t)T * H;
    if (int rc = ensure(g_arow, (size_t)T * A.rows * sizeof(float))) return rc;
    if (int rc = ensure(g_aqb, nth * hd * sizeof(float))) return rc;
    if (int rc = ensure(g_actx, nth * hd * sizeof(float))) return rc;
    if (!attn_uses_flash(T, hd)) {                    // (the flash kernel keeps no split partials)
        if (int rc = ensure(g_apo, nth * ns * hd * sizeof(float))) return rc;
        if (int rc = ensure(g_apml, nth * ns * 2 * sizeof(float))) return rc;
    }
    uint16_t *xb = nullptr;
    if (T > 4 && (A.nq > 0 || A.out_nq > 0)) {
        const size_t xbn = std::max(proj_xb_bytes(T, D, A.nq), proj_xb_bytes(T, A.qdim, A.out_nq));
        if (int rc = ensure(g_xb, xbn)) return rc;
        xb = static_cast<uint16_t *>(g_xb.p);
    }
    int img_tiles = 0;
    const size_t imgn = attn_flash_image_bytes(hd, d.n_kv, pos, T, &img_tiles);
    if (imgn)
        if (int rc = ensure(g_aimg, imgn)) return rc;
    float *rowb = static_cast<float *>(g_arow.p), *ctx = static_cast<float *>(g_actx.p);
    ProjArgs p{};
    p.counters = g_counters; p.ncounters = kCounters;
    p.x = x; p.ldx = D; p.y = rowb; p.ldy = A.rows; p.xb = xb; p.xb_n = xb ? g_xb.n : 0;
    p.Q = A.Qin; p.Qt = A.Qtin; p.scale = A.Sin; p.W = A.Win; p.T = T; p.I = D; p.O = A.rows; p.n_q = A.nq;
    HIP_OK(launch_proj(p, st));
    AttnArgs a{};
    a.qkv = rowb; a.ld_qkv = A.rows;
    a.qn = A.qn; a.kn = A.kn; a.inv = A.inv; a.Kc = A.Kc; a.Vc = A.Vc;
    a.qb = static_cast<float *>(g_aqb.p);
    a.po = static_cast<float *>(g_apo.p);
    a.pml = static_cast<float *>(g_apml.p);
    a.ctx = ctx;
    a.seq = seq; a.pos = pos; a.T = T; a.H = H; a.KV = d.n_kv; a.rot = d.rot_dim; a.max_t = d.max_t;
    a.ns = ns; a.kps = kps;
    a.eps = d.eps;
    a.scale = 1.f / sqrtf((float)hd);                // qwen.c:405
    a.img = imgn ? static_cast<unsigned char *>(g_aimg.p) : nullptr;
    a.img_tiles = img_tiles;
    HIP_OK(launch_attn(a, hd, st));
    ProjArgs q{};
    q.counters = g_counters; q.ncounters = kCounters;
    q.x = ctx; q.ldx = A.qdim; q.y = out; q.ldy = D; q.xb = xb; q.xb_n = xb ? g_xb.n : 0;
    q.Q = A.Qout; q.Qt = A.Qtout; q.scale = A.Sout; q.W = A.Wout; q.T = T; q.I = A.qdim; q.O = D; q.n_q = A.out_nq;
    HIP_OK(launch_proj(q, st));
    return OMH_OK;
}

}  // namespace

extern "C" {

int omh_init(void) {
    if (g_ready >= 0) return g_ready;
    g_ready = 0;
    const char *e = getenv("OM_HIP");
    if (e && e[0] == '0') { fail(OMH_ERR_DEVICE, "disabled by OM_HIP=0"); return 0; }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) { fail(OMH_ERR_DEVICE, "no HIP device"); return 0; }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) { fail(OMH_ERR_DEVICE, "hipGetDeviceProperties failed"); return 0; }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        fail(OMH_ERR_DEVICE, "device %d is %s, this library is built for gfx950", dev, prop.gcnArchName);
        return 0;
    }
    if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) {
        fail(OMH_ERR_DEVICE, "stream creation failed");
        return 0;
    }
    char *scr = nullptr;
    if (noalloc_scratch(&scr) != OMH_OK) return 0;        // the no-alloc scratch's device address
    if (hipMalloc(&g_counters, kCounters * sizeof(int)) != hipSuccess ||
        hipMemset(g_counters, 0, kCounters * sizeof(int)) != hipSuccess) {
        fail(OMH_ERR_DEVICE, "projection counters: allocation failed");
        return 0;
    }
    g_ready = 1;
    return 1;
}

const char *omh_last_error(void) { return g_err; }

int omh_gdn_layer_init(int li, const omh_gdn_dims *d, const omh_gdn_weights *w, int max_seqs) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (li < 0 || li >= kMaxLayers) return fail(OMH_ERR_ARG, "layer id %d outside [0, %d)", li, kMaxLayers);
    if (!d || !w || max_seqs < 1) return fail(OMH_ERR_ARG, "layer_init: null dims/weights or max_seqs < 1");
    if (d->kh < 1 || d->vh < d->kh || d->vh % d->kh || d->kd < 1 || d->vd < 1 || d->conv_k < 2)
        return fail(OMH_ERR_ARG, "layer_init: bad dims kh=%d vh=%d kd=%d vd=%d K=%d", d->kh, d->vh, d->kd, d->vd, d->conv_k);
    if (!decode_core_supported(d->kd, d->vd, d->vh / d->kh, d->conv_k))
        return fail(OMH_ERR_SHAPE, "layer_init: kd=%d vd=%d rep=%d K=%d unsupported", d->kd, d->vd,
                    d->vh / d->kh, d->conv_k);
    if (!w->conv_w || !w->A_log || !w->dt_bias || !w->gnorm) return fail(OMH_ERR_ARG, "layer_init: core weights missing");
    if (g_L[li].live) free_layer(g_L[li]);
    DevLayer L;
    L.d = *d;
    L.max_seqs = max_seqs;
    L.conv_dim = 2 * d->kh * d->kd + d->vh * d->vd;
    L.vdim = d->vh * d->vd;
    const int K = d->conv_k, D = d->hidden, vh = d->vh;
    int rc = OMH_OK;
#define UP(dst, n, src) do { if ((rc = upload(&(dst), (size_t)(n), (src))) != OMH_OK) { free_layer(L); return rc; } } while (0)
    {
        // device layout [conv_dim][kConvRing]: zeros, then taps 0..K-1
        std::vector<float> cw((size_t)L.conv_dim * kConvRing, 0.f);
        for (int c = 0; c < L.conv_dim; c++)
            for (int j = 0; j < K; j++) cw[(size_t)c * kConvRing + (kConvRing - K) + j] = w->conv_w[(size_t)c * K + j];
        UP(L.conv_w, cw.size(), cw.data());
    }
    UP(L.A_log, vh, w->A_log);
    UP(L.dt_bias, vh, w->dt_bias);
    UP(L.gnorm, d->vd, w->gnorm);
    const size_t nring = (size_t)max_seqs * L.conv_dim * kConvRing;
    const size_t nS = (size_t)max_seqs * vh * d->kd * d->vd;
    UP(L.conv_st, nring, (const float *)nullptr);
    UP(L.S, nS, (const float *)nullptr);
    UP(L.phase, (size_t)2 * max_seqs, (const int *)nullptr);
    UP(L.o_raw, (size_t)max_seqs * L.vdim, (const float *)nullptr);
    UP(L.ssq, (size_t)max_seqs * vh * kMaxSlices, (const float *)nullptr);
    UP(L.cnt, (size_t)max_seqs * vh, (const int *)nullptr);
    if (hipMemset(L.conv_st, 0, nring * sizeof(float)) != hipSuccess ||
        hipMemset(L.S, 0, nS * sizeof(float)) != hipSuccess ||
        hipMemset(L.phase, 0, 2 * max_seqs * sizeof(int)) != hipSuccess ||
        hipMemset(L.cnt, 0, (size_t)max_seqs * vh * sizeof(int)) != hipSuccess) {
        free_layer(L);
        return fail(OMH_ERR_DEVICE, "layer_init: state clear failed");
    }
    const bool any_proj = w->W_qkv || w->Q_qkv;
    if (any_proj) {
        const bool q8 = w->Q_qkv != nullptr;
        if (!proj_supported(D, q8 ? L.conv_dim + L.vdim : 0) || !proj_supported(L.vdim, w->Q_out ? D : 0)) {
            free_layer(L);
            return fail(OMH_ERR_SHAPE, "layer_init: projections need hidden and vh*vd multiples of 64 (got %d, %d)", D, L.vdim);
        }
        if (q8 && (!w->Q_z || !w->S_qkv || !w->S_z)) { free_layer(L); return fail(OMH_ERR_ARG, "layer_init: int8 in_proj needs Q_qkv, Q_z and their scales"); }
        if (!q8 && (!w->W_qkv || !w->W_z)) { free_layer(L); return fail(OMH_ERR_ARG, "layer_init: fp32 in_proj needs W_qkv and W_z"); }
        if (!w->W_b || !w->W_a) { free_layer(L); return fail(OMH_ERR_ARG, "layer_init: W_b and W_a are required"); }
        if (!w->Q_out && !w->W_out) { free_layer(L); return fail(OMH_ERR_ARG, "layer_init: out_proj missing"); }
        if (w->Q_out && !w->S_out) { free_layer(L); return fail(OMH_ERR_ARG, "layer_init: out_proj scales missing"); }
        L.in_rows = L.conv_dim + L.vdim + 2 * vh;
        const size_t Dz = (size_t)D;
        if (q8) {
            L.in_nq = L.conv_dim + L.vdim;
            std::vector<int8_t> q((size_t)L.in_nq * Dz);
            memcpy(q.data(), w->Q_qkv, (size_t)L.conv_dim * Dz);
            memcpy(q.data() + (size_t)L.conv_dim * Dz, w->Q_z, (size_t)L.vdim * Dz);
            std::vector<float> s(L.in_nq);
            memcpy(s.data(), w->S_qkv, L.conv_dim * sizeof(float));
            memcpy(s.data() + L.conv_dim, w->S_z, L.vdim * sizeof(float));
            UP(L.Qin, q.size(), q.data());
            UP(L.Sin, s.size(), s.data());
            if ((rc = upload_tiled(&L.Qtin, L.Qin, L.in_nq, D)) != OMH_OK) { free_layer(L); return rc; }
        }
        const int nf = L.in_rows - L.in_nq;
        std::vector<float> f((size_t)nf * Dz);
        size_t off = 0;
        if (!q8) {
            memcpy(f.data(), w->W_qkv, (size_t)L.conv_dim * Dz * sizeof(float)); off += (size_t)L.conv_dim * Dz;
            memcpy(f.data() + off, w->W_z, (size_t)L.vdim * Dz * sizeof(float)); off += (size_t)L.vdim * Dz;
        }
        memcpy(f.data() + off, w->W_b, (size_t)vh * Dz * sizeof(float)); off += (size_t)vh * Dz;
        memcpy(f.data() + off, w->W_a, (size_t)vh * Dz * sizeof(float));
        UP(L.Win, f.size(), f.data());
        if (w->Q_out) {
            L.out_nq = D;
            UP(L.Qout, (size_t)D * L.vdim, w->Q_out);
            UP(L.Sout, D, w->S_out);
            if ((rc = upload_tiled(&L.Qtout, L.Qout, D, L.vdim)) != OMH_OK) { free_layer(L); return rc; }
        } else {
            UP(L.Wout, (size_t)D * L.vdim, w->W_out);
        }
        L.has_proj = true;
    }
#undef UP
    L.live = true;
    g_L[li] = L;
    return OMH_OK;
}

int omh_gdn_layer_free(int li) {
    if (int rc = check_layer(li)) return rc;
    if (hipDeviceSynchronize() != hipSuccess) return fail(OMH_ERR_DEVICE, "layer_free: sync failed");
    free_layer(g_L[li]);
    return OMH_OK;
}

int omh_gdn_state_reset(int li, int seq) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    DevLayer &L = g_L[li];
    if (seq >= L.max_seqs) return fail(OMH_ERR_ARG, "state_reset: seq %d >= %d", seq, L.max_seqs);
    const size_t cn = (size_t)L.conv_dim * kConvRing, sn = (size_t)L.d.vh * L.d.kd * L.d.vd;
    const size_t s0 = seq < 0 ? 0 : (size_t)seq, ns = seq < 0 ? (size_t)L.max_seqs : 1;
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemset(L.conv_st + s0 * cn, 0, ns * cn * sizeof(float)));
    HIP_OK(hipMemset(L.S + s0 * sn, 0, ns * sn * sizeof(float)));
    HIP_OK(hipMemset(L.phase + (size_t)L.epoch * L.max_seqs + s0, 0, ns * sizeof(int)));
    HIP_OK(hipDeviceSynchronize());
    return OMH_OK;
}

int omh_gdn_state_get(int li, int seq, float *conv, float *S) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    DevLayer &L = g_L[li];
    if (seq < 0 || seq >= L.max_seqs) return fail(OMH_ERR_ARG, "state_get: seq %d outside [0, %d)", seq, L.max_seqs);
    const int K = L.d.conv_k;
    const size_t cn = (size_t)L.conv_dim * kConvRing, sn = (size_t)L.d.vh * L.d.kd * L.d.vd;
    HIP_OK(hipDeviceSynchronize());
    if (conv) {
        std::vector<float> ring(cn);
        int ph = 0;
        HIP_OK(hipMemcpy(ring.data(), L.conv_st + seq * cn, cn * sizeof(float), hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(&ph, L.phase + (size_t)L.epoch * L.max_seqs + seq, sizeof(int), hipMemcpyDeviceToHost));
        for (int c = 0; c < L.conv_dim; c++)
            for (int j = 0; j < K - 1; j++)
                conv[(size_t)c * (K - 1) + j] = ring[ring_at(0, ring_slot(ph, K, j), c, L.conv_dim)];
    }
    if (S) HIP_OK(hipMemcpy(S, L.S + seq * sn, sn * sizeof(float), hipMemcpyDeviceToHost));
    return OMH_OK;
}

int omh_gdn_state_set(int li, int seq, const float *conv, const float *S) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    DevLayer &L = g_L[li];
    if (seq < 0 || seq >= L.max_seqs) return fail(OMH_ERR_ARG, "state_set: seq %d outside [0, %d)", seq, L.max_seqs);
    const int K = L.d.conv_k;
    const size_t cn = (size_t)L.conv_dim * kConvRing, sn = (size_t)L.d.vh * L.d.kd * L.d.vd;
    HIP_OK(hipDeviceSynchronize());
    if (conv) {
        std::vector<float> ring(cn, 0.f);       // written at phase 0
        for (int c = 0; c < L.conv_dim; c++)
            for (int j = 0; j < K - 1; j++)
                ring[ring_at(0, ring_slot(0, K, j), c, L.conv_dim)] = conv[(size_t)c * (K - 1) + j];
        const int zero = 0;
        HIP_OK(hipMemcpy(L.conv_st + seq * cn, ring.data(), cn * sizeof(float), hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(L.phase + (size_t)L.epoch * L.max_seqs + seq, &zero, sizeof(int), hipMemcpyHostToDevice));
    }
    if (S) HIP_OK(hipMemcpy(L.S + seq * sn, S, sn * sizeof(float), hipMemcpyHostToDevice));
    return OMH_OK;
}

int omh_gdn_state_copy_dev(int nl, const int *lis, int src_seq, int dst_seq, void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (nl < 1 || !lis) return fail(OMH_ERR_ARG, "state_copy: nl=%d", nl);
    for (int i = 0; i < nl; i++) {
        if (int rc = check_layer(lis[i])) return rc;
        const DevLayer &L = g_L[lis[i]];
        if (src_seq < 0 || src_seq >= L.max_seqs || dst_seq < 0 || dst_seq >= L.max_seqs)
            return fail(OMH_ERR_ARG, "state_copy: sequences %d -> %d outside [0, %d) for layer %d", src_seq, dst_seq,
                        L.max_seqs, lis[i]);
        if (L.d.kh != g_L[lis[0]].d.kh || L.d.vh != g_L[lis[0]].d.vh || L.d.kd != g_L[lis[0]].d.kd ||
            L.d.vd != g_L[lis[0]].d.vd || L.conv_dim != g_L[lis[0]].conv_dim)
            return fail(OMH_ERR_ARG, "state_copy: layers %d and %d differ in shape", lis[0], lis[i]);
    }
    if (src_seq == dst_seq) return OMH_OK;
    const DevLayer &L0 = g_L[lis[0]];
    if ((L0.d.vh * L0.d.kd * L0.d.vd) % 4 != 0)
        return fail(OMH_ERR_SHAPE, "state_copy: vh*kd*vd = %d is not a multiple of 4", L0.d.vh * L0.d.kd * L0.d.vd);
    StateCopyArgs c{};
    c.n4 = (size_t)L0.d.vh * L0.d.kd * L0.d.vd / 4;
    c.r4 = (size_t)L0.conv_dim * kConvRing / 4;
    for (int l0 = 0; l0 < nl; l0 += kMaxDecodeLayers) {
        c.nl = nl - l0 < kMaxDecodeLayers ? nl - l0 : kMaxDecodeLayers;
        for (int j = 0; j < c.nl; j++) {
            const DevLayer &L = g_L[lis[l0 + j]];
            c.S_src[j] = L.S + (size_t)src_seq * c.n4 * 4;
            c.S_dst[j] = L.S + (size_t)dst_seq * c.n4 * 4;
            c.R_src[j] = L.conv_st + (size_t)src_seq * c.r4 * 4;
            c.R_dst[j] = L.conv_st + (size_t)dst_seq * c.r4 * 4;
            c.P_src[j] = L.phase + (size_t)L.epoch * L.max_seqs + src_seq;
            c.P_dst[j] = L.phase + (size_t)L.epoch * L.max_seqs + dst_seq;
        }
        HIP_OK(launch_state_copy(c, static_cast<hipStream_t>(stream)));
    }
    return OMH_OK;
}

int omh_gdn_state_copy(int nl, const int *lis, int src_seq, int dst_seq) {
    if (int rc = omh_gdn_state_copy_dev(nl, lis, src_seq, dst_seq, g_stream)) return rc;
    HIP_OK(hipStreamSynchronize(g_stream));
    return OMH_OK;
}

int omh_gdn_decode_core_seq_dev(int nl, const int *lis, int seq0, int B, const float *qkv, const float *z,
                                const float *a, const float *b, float *core, void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (nl < 1 || !lis) return fail(OMH_ERR_ARG, "decode_core_dev: nl=%d", nl);
    if (int rc = check_layer(lis[0])) return rc;
    const DevLayer &L = g_L[lis[0]];
    return decode_core(nl, lis, B, qkv, L.conv_dim, z, L.vdim, a, b, L.d.vh, core,
                       static_cast<hipStream_t>(stream), nullptr, seq0);
}

int omh_gdn_decode_core_dev(int nl, const int *lis, int B, const float *qkv, const float *z,
                            const float *a, const float *b, float *core, void *stream) {
    return omh_gdn_decode_core_seq_dev(nl, lis, 0, B, qkv, z, a, b, core, stream);
}

int omh_gdn_decode_core(int li, int B, const float *qkv, const float *z, const float *a,
                        const float *b, float *core) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    const DevLayer &L = g_L[li];
    if (B < 1 || B > L.max_seqs) return fail(OMH_ERR_ARG, "decode_core: B=%d outside [1, %d]", B, L.max_seqs);
    if (!qkv || !z || !a || !b || !core) return fail(OMH_ERR_ARG, "decode_core: null pointer");
    const size_t nq = (size_t)B * L.conv_dim, nz = (size_t)B * L.vdim, nab = (size_t)B * L.d.vh;
    if (int rc = ensure(g_qkv, nq * 4)) return rc;
    if (int rc = ensure(g_z, nz * 4)) return rc;
    if (int rc = ensure(g_a, nab * 4)) return rc;
    if (int rc = ensure(g_b, nab * 4)) return rc;
    if (int rc = ensure(g_core, nz * 4)) return rc;
    float *dq = (float *)g_qkv.p, *dz = (float *)g_z.p, *da = (float *)g_a.p, *db = (float *)g_b.p, *dc = (float *)g_core.p;
    HIP_OK(hipMemcpyAsync(dq, qkv, nq * 4, hipMemcpyHostToDevice, g_stream));
    HIP_OK(hipMemcpyAsync(dz, z, nz * 4, hipMemcpyHostToDevice, g_stream));
    HIP_OK(hipMemcpyAsync(da, a, nab * 4, hipMemcpyHostToDevice, g_stream));
    HIP_OK(hipMemcpyAsync(db, b, nab * 4, hipMemcpyHostToDevice, g_stream));
    if (int rc = decode_core(1, &li, B, dq, L.conv_dim, dz, L.vdim, da, db, L.d.vh, dc, g_stream)) return rc;
    HIP_OK(hipMemcpyAsync(core, dc, nz * 4, hipMemcpyDeviceToHost, g_stream));
    HIP_OK(hipStreamSynchronize(g_stream));
    return OMH_OK;
}

int omh_gdn_decode_dev(int li, int B, const float *x, float *out, void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    return decode_full(li, B, x, out, static_cast<hipStream_t>(stream));
}

int omh_gdn_decode_noalloc_dev(int li, int B, const float *x, float *out, void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = decode_full_args(li, B, x, out)) return rc;
    const size_t need = kNoAllocCounterBytes + decode_scratch(g_L[li], B).total;
    if (need > kNoAllocScratchBytes)
        return fail(OMH_ERR_SHAPE, "decode_noalloc: B=%d needs %zu bytes of scratch, above the %zu-byte static buffer",
                    B, need, kNoAllocScratchBytes);
    char *scr = nullptr;
    if (int rc = noalloc_scratch(&scr)) return rc;
    return decode_full_on(li, B, x, out, static_cast<hipStream_t>(stream), scr + kNoAllocCounterBytes,
                          reinterpret_cast<int *>(scr), (int)(kNoAllocCounterBytes / sizeof(int)));
}

int omh_gdn_decode(int li, int B, const float *x, float *out) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    const DevLayer &L = g_L[li];
    if (!L.has_proj) return fail(OMH_ERR_ARG, "layer %d was initialised without projections", li);
    if (B < 1 || B > L.max_seqs) return fail(OMH_ERR_ARG, "decode: B=%d outside [1, %d]", B, L.max_seqs);
    if (!x || !out) return fail(OMH_ERR_ARG, "decode: null pointer");
    const size_t n = (size_t)B * L.d.hidden;
    if (B <= 4 && n * 4 <= kPinnedMaxBytes) {
        if (int rc = stage_small(x, n, n)) return rc;
        if (int rc = decode_full(li, B, (const float *)g_x.p, g_hout.d, g_stream)) return rc;
        HIP_OK(hipStreamSynchronize(g_stream));
        memcpy(out, g_hout.h, n * 4);
        return OMH_OK;
    }
    if (int rc = ensure(g_x, n * 4)) return rc;
    if (int rc = ensure(g_out, n * 4)) return rc;
    HIP_OK(hipMemcpyAsync(g_x.p, x, n * 4, hipMemcpyHostToDevice, g_stream));
    if (int rc = decode_full(li, B, (const float *)g_x.p, (float *)g_out.p, g_stream)) return rc;
    HIP_OK(hipMemcpyAsync(out, g_out.p, n * 4, hipMemcpyDeviceToHost, g_stream));
    HIP_OK(hipStreamSynchronize(g_stream));
    return OMH_OK;
}

int omh_gdn_prefill(int li, int seq, int T, const float *x, float *out) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    const DevLayer &L = g_L[li];
    if (!L.has_proj) return fail(OMH_ERR_ARG, "layer %d was initialised without projections", li);
    if (T < 0 || (T > 0 && (!x || !out))) return fail(OMH_ERR_ARG, "prefill: bad arguments");
    if (T == 0) return OMH_OK;
    const size_t n = (size_t)T * L.d.hidden;
    if (int rc = ensure(g_x, n * 4)) return rc;
    if (int rc = ensure(g_out, n * 4)) return rc;
    HIP_OK(hipMemcpyAsync(g_x.p, x, n * 4, hipMemcpyHostToDevice, g_stream));
    if (int rc = prefill_full(li, seq, T, (const float *)g_x.p, (float *)g_out.p, g_stream)) return rc;
    HIP_OK(hipMemcpyAsync(out, g_out.p, n * 4, hipMemcpyDeviceToHost, g_stream));
    HIP_OK(hipStreamSynchronize(g_stream));
    return OMH_OK;
}

int omh_gdn_prefill_core(int li, int seq, int T, const float *qkv, const float *z, const float *a,
                         const float *b, float *core) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    const DevLayer &L = g_L[li];
    if (T < 0 || (T > 0 && (!qkv || !z || !a || !b || !core))) return fail(OMH_ERR_ARG, "prefill_core: bad arguments");
    if (T == 0) return OMH_OK;
    const size_t nq = (size_t)T * L.conv_dim, nz = (size_t)T * L.vdim, nab = (size_t)T * L.d.vh;
    if (int rc = ensure(g_qkv, nq * 4)) return rc;
    if (int rc = ensure(g_z, nz * 4)) return rc;
    if (int rc = ensure(g_a, nab * 4)) return rc;
    if (int rc = ensure(g_b, nab * 4)) return rc;
    if (int rc = ensure(g_core, nz * 4)) return rc;
    float *dq = (float *)g_qkv.p, *dz = (float *)g_z.p, *da = (float *)g_a.p, *db = (float *)g_b.p, *dc = (float *)g_core.p;
    HIP_OK(hipMemcpyAsync(dq, qkv, nq * 4, hipMemcpyHostToDevice, g_stream));
    HIP_OK(hipMemcpyAsync(dz, z, nz * 4, hipMemcpyHostToDevice, g_stream));
    HIP_OK(hipMemcpyAsync(da, a, nab * 4, hipMemcpyHostToDevice, g_stream));
    HIP_OK(hipMemcpyAsync(db, b, nab * 4, hipMemcpyHostToDevice, g_stream));
    if (int rc = prefill_core(li, seq, T, dq, L.conv_dim, dz, L.vdim, da, db, L.d.vh, dc, g_stream)) return rc;
    HIP_OK(hipMemcpyAsync(core, dc, nz * 4, hipMemcpyDeviceToHost, g_stream));
    HIP_OK(hipStreamSynchronize(g_stream));
    return OMH_OK;
}

int omh_gdn_prefill_core_dev(int li, int seq, int T, const float *qkv, const float *z, const float *a,
                             const float *b, float *core, void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_layer(li)) return rc;
    const DevLayer &L = g_L[li];
    return prefill_core(li, seq, T, qkv, L.conv_dim, z, L.vdim, a, b, L.d.vh, core, static_cast<hipStream_t>(stream));
}

int omh_gdn_prefill_dev(int li, int seq, int T, const float *x, float *out, void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    return prefill_full(li, seq, T, x, out, static_cast<hipStream_t>(stream));
}

int omh_sync(void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    HIP_OK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return OMH_OK;
}

int omh_attn_layer_init(int li, const omh_attn_dims *d, const omh_attn_weights *w, int max_seqs) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (li < 0 || li >= kMaxLayers) return fail(OMH_ERR_ARG, "attention layer id %d outside [0, %d)", li, kMaxLayers);
    if (!d || !w || max_seqs < 1) return fail(OMH_ERR_ARG, "attn_layer_init: null dims/weights or max_seqs < 1");
    if (d->hidden < 1 || d->n_heads < 1 || d->n_kv < 1 || d->head_dim < 1 || d->max_t < 1)
        return fail(OMH_ERR_ARG, "attn_layer_init: bad dims hidden=%d H=%d KV=%d hd=%d max_t=%d", d->hidden,
                    d->n_heads, d->n_kv, d->head_dim, d->max_t);
    if (!attn_supported(d->head_dim, d->n_heads, d->n_kv, d->rot_dim))
        return fail(OMH_ERR_SHAPE, "attn_layer_init: hd=%d H=%d KV=%d rot=%d unsupported", d->head_dim, d->n_heads,
                    d->n_kv, d->rot_dim);
    const bool q8 = w->Q_q != nullptr;
    if (q8 && (!w->Q_k || !w->Q_v || !w->S_q || !w->S_k || !w->S_v))
        return fail(OMH_ERR_ARG, "attn_layer_init: int8 q/k/v need Q_q, Q_k, Q_v and their scales");
    if (!q8 && (!w->W_q || !w->W_k || !w->W_v)) return fail(OMH_ERR_ARG, "attn_layer_init: fp32 q/k/v need W_q, W_k, W_v");
    if (!w->Q_o && !w->W_o) return fail(OMH_ERR_ARG, "attn_layer_init: o_proj missing");
    if (w->Q_o && !w->S_o) return fail(OMH_ERR_ARG, "attn_layer_init: o_proj scales missing");
    if (!w->q_norm || !w->k_norm) return fail(OMH_ERR_ARG, "attn_layer_init: q_norm and k_norm are required");
    const int D = d->hidden, H = d->n_heads, KV = d->n_kv, hd = d->head_dim;
    AttnLayer A;
    A.d = *d;
    A.max_seqs = max_seqs;
    A.qdim = H * hd;
    A.rows = 2 * H * hd + 2 * KV * hd;
    A.nq = q8 ? A.rows : 0;
    A.out_nq = w->Q_o ? D : 0;
    if (!proj_supported(D, A.nq) || !proj_supported(A.qdim, A.out_nq))
        return fail(OMH_ERR_SHAPE, "attn_layer_init: projections need hidden and H*hd multiples of 64 (got %d, %d)", D, A.qdim);
    if (g_A[li].live) free_attn(g_A[li]);
    int rc = OMH_OK;
#define UPA(dst, n, src) do { if ((rc = upload(&(dst), (size_t)(n), (src))) != OMH_OK) { free_attn(A); return rc; } } while (0)
    const size_t Dz = (size_t)D, nqr = (size_t)2 * H * hd, nkr = (size_t)KV * hd;
    if (q8) {
        std::vector<int8_t> q((size_t)A.rows * Dz);
        memcpy(q.data(), w->Q_q, nqr * Dz);
        memcpy(q.data() + nqr * Dz, w->Q_k, nkr * Dz);
        memcpy(q.data() + (nqr + nkr) * Dz, w->Q_v, nkr * Dz);
        std::vector<float> s(A.rows);
        memcpy(s.data(), w->S_q, nqr * sizeof(float));
        memcpy(s.data() + nqr, w->S_k, nkr * sizeof(float));
        memcpy(s.data() + nqr + nkr, w->S_v, nkr * sizeof(float));
        UPA(A.Qin, q.size(), q.data());
        UPA(A.Sin, s.size(), s.data());
        if ((rc = upload_tiled(&A.Qtin, A.Qin, A.rows, D)) != OMH_OK) { free_attn(A); return rc; }
    } else {
        std::vector<float> f((size_t)A.rows * Dz);
        memcpy(f.data(), w->W_q, nqr * Dz * sizeof(float));
        memcpy(f.data() + nqr * Dz, w->W_k, nkr * Dz * sizeof(float));
        memcpy(f.data() + (nqr + nkr) * Dz, w->W_v, nkr * Dz * sizeof(float));
        UPA(A.Win, f.size(), f.data());
    }
    if (w->Q_o) {
        UPA(A.Qout, (size_t)D * A.qdim, w->Q_o);
        UPA(A.Sout, D, w->S_o);
        if ((rc = upload_tiled(&A.Qtout, A.Qout, D, A.qdim)) != OMH_OK) { free_attn(A); return rc; }
    } else {
        UPA(A.Wout, (size_t)D * A.qdim, w->W_o);
    }
    UPA(A.qn, hd, w->q_norm);
    UPA(A.kn, hd, w->k_norm);
    {
        // RoPE inverse frequencies, the engine's expression (qwen.c:392)
        const int half = d->rot_dim / 2;
        std::vector<float> inv(half > 0 ? half : 1, 0.f);
        for (int j = 0; j < half; j++) inv[j] = powf(d->theta, -(float)(2 * j) / (float)d->rot_dim);
        UPA(A.inv, inv.size(), inv.data());
    }
    const size_t nc = (size_t)max_seqs * KV * d->max_t * hd;
    UPA(A.Kc, nc, (const float *)nullptr);
    UPA(A.Vc, nc, (const float *)nullptr);
    if (hipMemset(A.Kc, 0, nc * sizeof(float)) != hipSuccess || hipMemset(A.Vc, 0, nc * sizeof(float)) != hipSuccess) {
        free_attn(A);
        return fail(OMH_ERR_DEVICE, "attn_layer_init: cache clear failed");
    }
#undef UPA
    A.live = true;
    g_A[li] = A;
    return OMH_OK;
}

int omh_attn_layer_free(int li) {
    if (int rc = check_attn(li)) return rc;
    if (hipDeviceSynchronize() != hipSuccess) return fail(OMH_ERR_DEVICE, "attn_layer_free: sync failed");
    free_attn(g_A[li]);
    return OMH_OK;
}

// Rows t0 .. t0+n-1 of every kv head of one sequence's K and V caches,
// to or from host arrays in the engine's layout [n_kv][ld_t][head_dim]
// (m->K[li], m->V[li] with ld_t = m->max_t, engines/qwen.c:257-258, 399-402).
static int attn_cache_copy(int li, int seq, int t0, int n, float *K, float *V, int ld_t, bool to_host) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_attn(li)) return rc;
    const AttnLayer &A = g_A[li];
    const omh_attn_dims &d = A.d;
    if (seq < 0 || seq >= A.max_seqs) return fail(OMH_ERR_ARG, "attn cache: seq %d outside [0, %d)", seq, A.max_seqs);
    if (t0 < 0 || n < 0 || (long)t0 + n > d.max_t || (long)t0 + n > ld_t)
        return fail(OMH_ERR_ARG, "attn cache: rows %d..%d outside the cache of %d (host rows %d)", t0, t0 + n - 1,
                    d.max_t, ld_t);
    if (n == 0) return OMH_OK;
    // Work a caller enqueued on its own streams (omh_attn_forward_dev) may
    // still be writing or reading these rows: wait for the whole device
    // first, as omh_gdn_state_get / _set do.
    HIP_OK(hipDeviceSynchronize());
    const size_t hd = d.head_dim, row = hd * sizeof(float), w = (size_t)n * row;
    for (int h = 0; h < d.n_kv; h++) {
        const size_t dev_off = (((size_t)seq * d.n_kv + h) * d.max_t + t0) * hd;
        const size_t host_off = ((size_t)h * ld_t + t0) * hd;
        float *dk = A.Kc + dev_off, *dv = A.Vc + dev_off;
        if (to_host) {
            if (K) HIP_OK(hipMemcpyAsync(K + host_off, dk, w, hipMemcpyDeviceToHost, g_stream));
            if (V) HIP_OK(hipMemcpyAsync(V + host_off, dv, w, hipMemcpyDeviceToHost, g_stream));
        } else {
            if (K) HIP_OK(hipMemcpyAsync(dk, K + host_off, w, hipMemcpyHostToDevice, g_stream));
            if (V) HIP_OK(hipMemcpyAsync(dv, V + host_off, w, hipMemcpyHostToDevice, g_stream));
        }
    }
    HIP_OK(hipStreamSynchronize(g_stream));
    return OMH_OK;
}

int omh_attn_cache_get(int li, int seq, int t0, int n, float *K, float *V, int ld_t) {
    return attn_cache_copy(li, seq, t0, n, K, V, ld_t, true);
}

int omh_attn_cache_set(int li, int seq, int t0, int n, const float *K, const float *V, int ld_t) {
    return attn_cache_copy(li, seq, t0, n, const_cast<float *>(K), const_cast<float *>(V), ld_t, false);
}

int omh_attn_forward_dev(int li, int seq, int pos, int T, const float *x, float *out, void *stream) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    return attn_forward(li, seq, pos, T, x, out, static_cast<hipStream_t>(stream));
}

int omh_attn_forward(int li, int seq, int pos, int T, const float *x, float *out) {
    if (!omh_init()) return OMH_ERR_DEVICE;
    if (int rc = check_attn(li)) return rc;
    if (T < 0 || (T > 0 && (!x || !out))) return fail(OMH_ERR_ARG, "attn: bad arguments");
    if (T == 0) return OMH_OK;
    const size_t n = (size_t)T * g_A[li].d.hidden;
    if (T <= 4 && n * 4 <= kPinnedMaxBytes) {      // the engine's decode step (o_proj on the GEMV)
        if (int rc = stage_small(x, n, n)) return rc;
        if (int rc = attn_forward(li, seq, pos, T, (const float *)g_x.p, g_hout.d, g_stream)) return rc;
        HIP_OK(hipStreamSynchronize(g_stream));
        memcpy(out, g_hout.h, n * 4);
        return OMH_OK;
    }
    if (int rc = ensure(g_x, n * 4)) return rc;
    if (int rc = ensure(g_out, n * 4)) return rc;
    HIP_OK(hipMemcpyAsync(g_x.p, x, n * 4, hipMemcpyHostToDevice, g_stream));
    if (int rc = attn_forward(li, seq, pos, T, (const float *)g_x.p, (float *)g_out.p, g_stream)) return rc;
    HIP_OK(hipMemcpyAsync(out, g_out.p, n * 4, hipMemcpyDeviceToHost, g_stream));
    HIP_OK(hipStreamSynchronize(g_stream));
    return OMH_OK;
}

}  // extern "C"
