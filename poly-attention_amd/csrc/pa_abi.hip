// pa_abi.hip -- the extern "C" entry points of libpolyattn.so: argument validation and
// kernel dispatch.  Declarations and semantics: include/polyattn.h.
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "pa_common.h"
#include "pa_launch.h"

namespace pa {

// Process-wide: torch runs a backward pass on its own autograd thread, so the recording
// state cannot be thread-local.
struct ProfRec {
    const char* name;
    hipEvent_t start, stop;
};
static std::atomic<bool> g_prof_on{false};
static std::mutex g_prof_mu;
static std::vector<ProfRec> g_prof;

ProfScope::ProfScope(const char* name, hipStream_t s) : active(false), idx(0), stream(s) {
    if (!g_prof_on.load(std::memory_order_relaxed)) return;
    ProfRec r{name, nullptr, nullptr};
    if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) return;
    (void)hipEventRecord(r.start, s);
    std::lock_guard<std::mutex> lock(g_prof_mu);
    idx = g_prof.size();
    g_prof.push_back(r);
    active = true;
}

ProfScope::~ProfScope() {
    if (!active) return;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    (void)hipEventRecord(g_prof[idx].stop, stream);
}

}  // namespace pa

using namespace pa;

namespace {

thread_local int g_last_hip_error = 0;

bool valid_dtype(int d) { return d == PA_F32 || d == PA_F16 || d == PA_BF16; }

// A view that is either absent (allowed when !required) or well-formed for a pass with
// `pass_heads` heads.  want_dtype < 0 accepts any element type.
int check_view(const pa_view& v, int pass_heads, bool required, int want_dtype) {
    if (!v.ptr) return required ? PA_EINVAL : PA_OK;
    if (v.heads <= 0 || pass_heads % v.heads != 0) return PA_EINVAL;
    if (!valid_dtype(v.dtype)) return PA_EINVAL;
    if (want_dtype >= 0 && v.dtype != want_dtype) return PA_EINVAL;
    return PA_OK;
}

DView to_dview(const pa_view& v, int pass_heads) {
    DView d;
    d.p = static_cast<char*>(v.ptr);
    d.sb = v.sb;
    d.sh = v.sh;
    d.sn = v.sn;
    d.hdiv = (v.ptr && v.heads > 0) ? pass_heads / v.heads : 1;
    d.dtype = v.dtype;
    return d;
}

DMask to_dmask(const pa_mask& m) {
    DMask d;
    d.p = m.ptr;
    d.sb = m.sb;
    d.sn = m.sn;
    return d;
}

#define PA_TRY(expr)                   \
    do {                               \
        int _st = (expr);              \
        if (_st != PA_OK) return _st;  \
    } while (0)

int validate_pass(const pa_pass* p) {
    if (!p) return PA_EINVAL;
    if (p->batch < 1 || p->heads < 1 || p->nq < 1 || p->nk < 1) return PA_EINVAL;
    if (p->dim < 1 || p->dim > 256) return PA_EUNSUPPORTED;
    const int T = p->q.dtype;
    if (!valid_dtype(T)) return PA_EINVAL;
    PA_TRY(check_view(p->q, p->heads, true, T));
    PA_TRY(check_view(p->k, p->heads, true, T));
    PA_TRY(check_view(p->v, p->heads, true, T));
    PA_TRY(check_view(p->vmul, p->heads, false, T));
    PA_TRY(check_view(p->bias, p->heads, false, -1));
    PA_TRY(check_view(p->out, p->heads, true, T));
    PA_TRY(check_view(p->lse, p->heads, true, PA_F32));
    if (p->out.heads != p->heads || p->lse.heads != p->heads) return PA_EINVAL;
    if (p->epi) {
        const pa_epilogue* e = p->epi;
        PA_TRY(check_view(e->root, p->heads, false, T));
        PA_TRY(check_view(e->gate, p->heads, false, T));
        PA_TRY(check_view(e->y, p->heads, true, T));
        if (e->y.heads != p->heads || (e->gate.ptr && e->gate.heads != p->heads)) return PA_EINVAL;
        if (e->flags & ~PA_EPI_ROOT_SIGMOID) return PA_EINVAL;
    }
    return PA_OK;
}

PassDev to_passdev(const pa_pass* p) {
    PassDev P;
    P.batch = p->batch;
    P.heads = p->heads;
    P.nq = p->nq;
    P.nk = p->nk;
    P.dim = p->dim;
    P.scale = p->scale;
    P.softclamp = p->softclamp;
    P.causal = p->causal;
    P.flags = p->flags;
    P.q = to_dview(p->q, p->heads);
    P.k = to_dview(p->k, p->heads);
    P.v = to_dview(p->v, p->heads);
    P.vmul = to_dview(p->vmul, p->heads);
    P.bias = to_dview(p->bias, p->heads);
    P.out = to_dview(p->out, p->heads);
    P.lse = to_dview(p->lse, p->heads);
    P.km = to_dmask(p->key_mask);
    P.qm = to_dmask(p->query_mask);
    const pa_view none = {};
    const pa_epilogue* e = p->epi;
    P.er = to_dview(e ? e->root : none, p->heads);
    P.eg = to_dview(e ? e->gate : none, p->heads);
    P.ey = to_dview(e ? e->y : none, p->heads);
    P.eflags = e ? e->flags : 0;
    const pa_qk_norm* n = p->norm;
    P.nflags = n ? n->flags : 0;
    P.qnw = n ? n->q_weight : nullptr;
    P.knw = n ? n->k_weight : nullptr;
    P.qeps = n ? n->q_eps : 0.f;
    P.keps = n ? n->k_eps : 0.f;
    P.live = nullptr;
    return P;
}

int finish_launch() {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_last_hip_error = static_cast<int>(e);
        return PA_EHIP;
    }
    return PA_OK;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// The MFMA backward of a masked pass runs on the pass without its masks (the key mask folded
// into the key term, fully-masked rows given lse = +inf and finished by the fix-ups): whether
// the kernels take that mask-free pass.
bool mfma_bwd_masked_supported(const GradDev& G, int dtype) {
    GradDev Gm = G;
    Gm.f.km.p = nullptr;
    Gm.f.qm.p = nullptr;
    Gm.f.flags &= ~PA_FLAG_MAY_DEGENERATE;
    return mfma_bwd_supported(Gm, dtype);
}

bool pass_masked(const pa_pass& f) {
    return f.key_mask.ptr || f.query_mask.ptr || (f.flags & PA_FLAG_MAY_DEGENERATE);
}

// key-term row stride: whole 16-byte chunks
int key_term_stride(const pa_pass& f) { return (f.nk + 3) & ~3; }

size_t elem_bytes(int dtype) { return dtype == PA_F32 ? 4 : 2; }

// forward workspace: the per-key term of a key-masked 16-bit pass on the MFMA kernels, whose
// key bias it then is, and the range of keys that can enter a normal row
size_t fwd_ws_bytes(const pa_pass& f) {
    if (!f.key_mask.ptr || (f.q.dtype != PA_BF16 && f.q.dtype != PA_F16)) return 0;
    if (f.dim != 64 && f.dim != 128) return 0;
    if (f.bias.ptr && f.bias.heads != f.k.heads) return 0;  // one key term per key head
    const size_t kheads = (size_t)f.batch * f.k.heads;
    return align256(kheads * key_term_stride(f) * sizeof(float)) +
           align256(kheads * 2 * sizeof(int32_t));
}

// [D | lse | 1/c1] per query row; with an epilogue the gradient reaching the pass output;
// masked passes add the key term (with a key mask), the per-head fully-masked-row sums, the
// per-key-head bias-class counts and the per-key-head range of keys that can enter a normal row
size_t bwd_ws_bytes(const pa_pass& f) {
    const size_t rows = (size_t)f.batch * f.heads * f.nq;
    size_t n = 3 * align256(rows * sizeof(float));
    if (f.epi) n += align256(rows * f.dim * elem_bytes(f.q.dtype));
    if (pass_masked(f)) {
        const size_t kheads = (size_t)f.batch * f.k.heads;
        if (f.key_mask.ptr) n += align256(kheads * key_term_stride(f) * sizeof(float));
        n += align256((size_t)f.batch * f.heads * fix_row_chunks(f.nq) * (f.dim + 2) * sizeof(float));
        n += 2 * align256(kheads * 2 * sizeof(int32_t));
    }
    return n;
}

}  // namespace

extern "C" {

int pa_abi_version(void) { return PA_ABI_VERSION; }

const char* pa_strerror(int status) {
    switch (status) {
        case PA_OK: return "success";
        case PA_EINVAL: return "invalid argument (shape, stride, head count, dtype or pointer)";
        case PA_EUNSUPPORTED: return "unsupported by this build of libpolyattn";
        case PA_EHIP: return "HIP runtime error";
        case PA_EWORKSPACE: return "workspace missing or too small";
        case PA_ESCRATCH:
            return "the request needs more split-K scratch than the library's static "
                   "PA_DECODE_SCRATCH_BYTES per device (use pa_poly_decode with a workspace)";
        default: return "unknown libpolyattn status";
    }
}

int pa_last_hip_error(void) { return g_last_hip_error; }

size_t pa_struct_size(int which) {
    switch (which) {
        case 0: return sizeof(pa_view);
        case 1: return sizeof(pa_mask);
        case 2: return sizeof(pa_pass);
        case 3: return sizeof(pa_pass_grad);
        case 4: return sizeof(pa_decode_level);
        case 5: return sizeof(pa_decode);
        case 6: return sizeof(pa_prologue_item);
        case 7: return sizeof(pa_prologue);
        case 8: return sizeof(pa_rmsnorm);
        case 9: return sizeof(pa_linear);
        case 10: return sizeof(pa_linear_out);
        case 11: return sizeof(pa_epilogue);
        case 12: return sizeof(pa_qk_norm);
        default: return 0;
    }
}

int pa_profile_start(void) {
    std::lock_guard<std::mutex> lock(g_prof_mu);
    for (ProfRec& r : g_prof) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    g_prof.clear();
    g_prof_on = true;
    return PA_OK;
}

int pa_profile_stop(pa_kernel_time* out, int capacity, int* count) {
    g_prof_on = false;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    int n = 0;
    int status = PA_OK;
    for (ProfRec& r : g_prof) {
        float ms = 0.f;
        if (hipEventSynchronize(r.stop) != hipSuccess ||
            hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) {
            status = PA_EHIP;
        }
        int k = 0;
        while (k < n && std::strcmp(out[k].name, r.name) != 0) ++k;
        if (k == n) {
            if (n >= capacity) continue;
            out[n].name = r.name;
            out[n].launches = 0;
            out[n].total_ms = 0.0;
            ++n;
        }
        out[k].launches += 1;
        out[k].total_ms += ms;
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    g_prof.clear();
    if (count) *count = n;
    return status;
}

// ---------------------------------------------------------------------------------------
// Clock probe: 256 workgroups of 8 waves (two per SIMD), each wave four independent MFMA chains
// of kClkIters products bracketed by s_memtime (shader cycles) and s_memrealtime (100 MHz).
// Lanes 0 and 1 of every wave store its two counts (per-lane addresses: vector stores).
constexpr int kClkWgs = 256, kClkWaves = 8, kClkIters = 768;
__device__ unsigned long long g_clk[kClkWgs * kClkWaves * 2];

__global__ __launch_bounds__(64 * kClkWaves) void k_clock_probe() {
    typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
    typedef float f16v __attribute__((ext_vector_type(16)));
    bf8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(threadIdx.x * 1e-3f);
        b[i] = (__bf16)(i * 1e-2f);
    }
    f16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < kClkIters / 4; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
    }
    float sum = 0.f;
    for (int i = 0; i < 16; ++i) sum += c0[i] + c1[i] + c2[i] + c3[i];
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    const int lane = threadIdx.x & 63, wave = blockIdx.x * kClkWaves + (threadIdx.x >> 6);
    // (the sum keeps the chains live: it is never NaN for these inputs, so both counts store)
    if (lane < 2 && !(sum != sum)) g_clk[wave * 2 + lane] = lane == 0 ? t1 - t0 : r1 - r0;
}

int pa_measure_clock(double* ghz, void* stream) {
    if (!ghz) return PA_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<unsigned long long> host(kClkWgs * kClkWaves * 2);
    hipLaunchKernelGGL(k_clock_probe, dim3(kClkWgs), dim3(64 * kClkWaves), 0, s);
    if (hipGetLastError() != hipSuccess) return PA_EHIP;
    if (hipStreamSynchronize(s) != hipSuccess) return PA_EHIP;
    if (hipMemcpyFromSymbol(host.data(), HIP_SYMBOL(g_clk), host.size() * sizeof(host[0]), 0,
                            hipMemcpyDeviceToHost) != hipSuccess)
        return PA_EHIP;
    double cyc = 0.0, ticks = 0.0;
    for (int w = 0; w < kClkWgs * kClkWaves; ++w) {
        cyc += (double)host[2 * w];
        ticks += (double)host[2 * w + 1];
    }
    if (!(ticks > 0.0)) return PA_EHIP;
    *ghz = cyc / ticks * 0.1;  // cycles per 10 ns tick -> GHz
    return PA_OK;
}

size_t pa_attn_pass_fwd_workspace(const pa_pass* p) { return p ? fwd_ws_bytes(*p) : 0; }

// q / k norms on load: valid flags and weights, and only where the short-pass kernel runs
static int check_norm(const pa_pass* p, const PassDev& P) {
    if (!P.nflags) return PA_OK;
    const pa_qk_norm* n = p->norm;
    if (n->flags & ~(PA_NORM_Q | PA_NORM_K)) return PA_EINVAL;
    if (((n->flags & PA_NORM_Q) && (!n->q_weight || (uintptr_t)n->q_weight % 16)) ||
        ((n->flags & PA_NORM_K) && (!n->k_weight || (uintptr_t)n->k_weight % 16)))
        return PA_EINVAL;
    const int T = p->q.dtype;
    if (!mfma_fwd_supported(P, T) || !mfma_fwd_short_applies(P, T)) return PA_EUNSUPPORTED;
    return PA_OK;
}

int pa_attn_pass_fwd(const pa_pass* p, void* stream) {
    PA_TRY(validate_pass(p));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const PassDev P = to_passdev(p);
    const int T = p->q.dtype;
    PA_TRY(check_norm(p, P));
    if (mfma_fwd_supported(P, T)) {
        const size_t need = fwd_ws_bytes(*p);
        if (need && p->workspace && p->workspace_bytes >= need) {
            // the key mask folded into a per-key term read as the key bias (the
            // direct-to-LDS kernel has no key-mask path); fully-masked rows as before
            const int hk = p->k.heads, nkp = key_term_stride(*p);
            char* w = static_cast<char*>(p->workspace);
            float* kterm = reinterpret_cast<float*>(w);
            GradDev G = {};  // the key-term kernel reads f and hk only
            G.f = P;
            G.hk = hk;
            int32_t* live = reinterpret_cast<int32_t*>(
                w + align256((size_t)p->batch * hk * nkp * sizeof(float)));
            launch_key_terms(G, kterm, nkp, nullptr, live, s);  // the counts serve the backward
            PassDev Pm = P;
            Pm.bias = DView{reinterpret_cast<char*>(kterm), (int64_t)hk * nkp, nkp, 1,
                            p->heads / hk, PA_F32};
            Pm.km.p = nullptr;
            Pm.live = live;
            launch_mfma_fwd(Pm, T, s);
        } else {
            launch_mfma_fwd(P, T, s);
        }
        const bool may_degenerate = (p->flags & PA_FLAG_MAY_DEGENERATE) || p->key_mask.ptr ||
                                    p->query_mask.ptr;
        if (may_degenerate) launch_fwd_fixup(P, T, s);
    } else {
        launch_simt_fwd(P, T, s);
    }
    return finish_launch();
}

static bool same_view(const pa_view& a, const pa_view& b) {
    return a.ptr == b.ptr && a.sb == b.sb && a.sh == b.sh && a.sn == b.sn && a.heads == b.heads &&
           a.dtype == b.dtype;
}

int pa_poly_order2_fwd(const pa_pass* first, const pa_pass* second, void* stream) {
    PA_TRY(validate_pass(first));
    PA_TRY(validate_pass(second));
    // the chain: the second pass's keys, values and key term are the first's queries, output
    // and lse
    if (!same_view(second->k, first->q) || !same_view(second->v, first->out) ||
        !same_view(second->bias, first->lse) || second->nk != first->nq)
        return PA_EINVAL;
    const PassDev P1 = to_passdev(first), P2 = to_passdev(second);
    PA_TRY(check_norm(first, P1));
    PA_TRY(check_norm(second, P2));
    const int T = first->q.dtype;
    const bool degenerate = ((first->flags | second->flags) & PA_FLAG_MAY_DEGENERATE) != 0;
    if (!degenerate && second->q.dtype == T && mfma_order2_short_applies(P1, P2, T)) {
        launch_order2_short(P1, P2, T, static_cast<hipStream_t>(stream));
        return finish_launch();
    }
    PA_TRY(pa_attn_pass_fwd(first, stream));
    return pa_attn_pass_fwd(second, stream);
}

size_t pa_attn_pass_bwd_workspace(const pa_pass_grad* g) {
    if (!g) return 0;
    return bwd_ws_bytes(g->fwd);
}

int pa_attn_pass_bwd(const pa_pass_grad* g, void* stream) {
    if (!g) return PA_EINVAL;
    const pa_pass* p = &g->fwd;
    PA_TRY(validate_pass(p));
    if (p->norm && p->norm->flags) return PA_EUNSUPPORTED;  // forward only
    const int T = p->q.dtype;
    const int H = p->heads;
    const int hk = p->k.heads;
    // backward: queries at the pass head count, key-side tensors at one head count
    if (p->q.heads != H) return PA_EUNSUPPORTED;
    if (p->v.heads != hk) return PA_EUNSUPPORTED;
    if (p->vmul.ptr && p->vmul.heads != hk) return PA_EUNSUPPORTED;
    if (p->bias.ptr && p->bias.heads != hk) return PA_EUNSUPPORTED;
    PA_TRY(check_view(g->dout, H, true, T));
    PA_TRY(check_view(g->dlse, H, false, PA_F32));
    PA_TRY(check_view(g->dq, H, true, T));
    PA_TRY(check_view(g->dk, H, true, T));
    PA_TRY(check_view(g->dv, H, true, T));
    PA_TRY(check_view(g->dvmul, H, p->vmul.ptr != nullptr, T));
    PA_TRY(check_view(g->dbias, H, false, PA_F32));
    if (g->dout.heads != H || g->dq.heads != H || g->dk.heads != hk || g->dv.heads != hk)
        return PA_EINVAL;
    if (g->dvmul.ptr && g->dvmul.heads != hk) return PA_EINVAL;
    if (g->dbias.ptr && g->dbias.heads != hk) return PA_EINVAL;
    if (g->dlse.ptr && g->dlse.heads != H) return PA_EINVAL;
    if (p->epi) {
        PA_TRY(check_view(g->droot, H, p->epi->root.ptr != nullptr, T));
        PA_TRY(check_view(g->dgate, H, p->epi->gate.ptr != nullptr, T));
        if (g->droot.ptr && g->droot.heads != p->epi->root.heads) return PA_EINVAL;
        if (g->dgate.ptr && g->dgate.heads != H) return PA_EINVAL;
    }
    const size_t need = bwd_ws_bytes(*p);
    if (!g->workspace || g->workspace_bytes < need) return PA_EWORKSPACE;

    GradDev G;
    G.f = to_passdev(p);
    G.dout = to_dview(g->dout, H);
    G.dlse = to_dview(g->dlse, H);
    G.dq = to_dview(g->dq, H);
    G.dk = to_dview(g->dk, H);
    G.dv = to_dview(g->dv, H);
    G.dvmul = to_dview(g->dvmul, H);
    G.dbias = to_dview(g->dbias, H);
    G.accumulate = g->accumulate;
    G.hk = hk;
    const size_t rows = (size_t)p->batch * H * p->nq;
    char* ws = static_cast<char*>(g->workspace);
    G.ws_D = reinterpret_cast<float*>(ws);
    G.ws_lse = reinterpret_cast<float*>(ws + align256(rows * sizeof(float)));
    G.ws_invc = reinterpret_cast<float*>(ws + 2 * align256(rows * sizeof(float)));
    ws += 3 * align256(rows * sizeof(float));
    const pa_view none = {};
    G.droot = to_dview(p->epi ? g->droot : none, H);
    G.dgate = to_dview(p->epi ? g->dgate : none, H);

    hipStream_t s = static_cast<hipStream_t>(stream);
    if (p->epi) {
        // the epilogue's gradients, and the gradient reaching the pass output (dO) in the
        // workspace, which the pass backward then reads as its dout
        char* dO = ws;
        ws += align256(rows * p->dim * elem_bytes(T));
        const int hr = p->epi->root.ptr ? p->epi->root.heads : H;
        launch_epi_bwd(G, dO, hr, T, s);
        DView& d = G.dout;
        d.p = dO;
        d.sn = p->dim;
        d.sh = (int64_t)p->nq * p->dim;
        d.sb = (int64_t)H * d.sh;
        d.hdiv = 1;
        d.dtype = T;
    }
    G.fused_pre = 0;
    G.seeds = 0;
    G.ws_kcnt = nullptr;
    G.ws_part = nullptr;
    if (pass_masked(*p) && mfma_bwd_masked_supported(G, T)) {
        // normal rows on the MFMA kernels with the key mask folded into the key bias; the
        // preprocess marks fully-masked rows (lse = +inf), whose part the fix-ups add
        char* w = ws;
        float* kterm = nullptr;
        const int nkp = key_term_stride(*p);
        if (p->key_mask.ptr) {
            kterm = reinterpret_cast<float*>(w);
            w += align256((size_t)p->batch * hk * nkp * sizeof(float));
        }
        G.ws_part = reinterpret_cast<float*>(w);
        w += align256((size_t)p->batch * H * fix_row_chunks(p->nq) * (p->dim + 2) * sizeof(float));
        int32_t* kcnt = reinterpret_cast<int32_t*>(w);
        w += align256((size_t)p->batch * hk * 2 * sizeof(int32_t));
        int32_t* live = reinterpret_cast<int32_t*>(w);
        G.ws_kcnt = kcnt;
        launch_key_terms(G, kterm, nkp, kcnt, live, s);
        GradDev Gm = G;
        if (kterm) {
            DView& kb = Gm.f.bias;
            kb.p = reinterpret_cast<char*>(kterm);
            kb.sb = (int64_t)hk * nkp;
            kb.sh = nkp;
            kb.sn = 1;
            kb.hdiv = H / hk;
            kb.dtype = PA_F32;
        }
        Gm.f.km.p = nullptr;
        Gm.f.qm.p = nullptr;
        Gm.f.flags &= ~PA_FLAG_MAY_DEGENERATE;
        Gm.f.live = live;
        // the direct-to-LDS dQ kernel does the preprocess of the normal rows where it applies
        // (fully-masked rows get lse +inf there: no normal entry; k_fix_rows does the rest of
        // their preprocess from the original masks)
        Gm.fused_pre = mfma_bwd_fuses_pre(Gm) ? 1 : 0;
        if (!Gm.fused_pre) launch_simt_bwd(G, T, s, /*pre=*/true, false, false);
        launch_mfma_bwd(Gm, T, s);
        launch_mask_fixups(G, T, s);
    } else if (mfma_bwd_supported(G, T)) {
        // the direct-to-LDS dQ kernel computes the per-row preprocess itself when it applies
        G.fused_pre = mfma_bwd_fuses_pre(G) ? 1 : 0;
        if (!G.fused_pre) launch_simt_bwd(G, T, s, /*pre=*/true, false, false);
        launch_mfma_bwd(G, T, s);
    } else {
        launch_simt_bwd(G, T, s, /*pre=*/true, false, false);
        launch_simt_bwd(G, T, s, false, /*dq=*/true, /*dkv=*/true);
    }
    return finish_launch();
}

size_t pa_poly_decode_workspace(const pa_decode* d) {
    if (!d) return 0;
    int chunk = 0, nchunks = 0;
    return decode_workspace_bytes(d, &chunk, &nchunks);
}

int pa_poly_decode(const pa_decode* d, void* stream) {
    if (!d) return PA_EINVAL;
    const int st = launch_decode(d, static_cast<hipStream_t>(stream));
    if (st != PA_OK) return st;
    return finish_launch();
}

int pa_poly_decode_noalloc(const pa_decode* d, void* stream) {
    if (!d) return PA_EINVAL;
    int hip_err = 0;
    const int st = launch_decode_noalloc(d, static_cast<hipStream_t>(stream), &hip_err);
    if (st == PA_EHIP) g_last_hip_error = hip_err;
    if (st != PA_OK) return st;
    return finish_launch();
}

int pa_decode_prologue(const pa_prologue* p, void* stream) {
    if (!p) return PA_EINVAL;
    const int st = launch_prologue(p, static_cast<hipStream_t>(stream));
    if (st != PA_OK) return st;
    return finish_launch();
}

int pa_rmsnorm_fwd(const pa_rmsnorm* r, void* stream) {
    if (!r) return PA_EINVAL;
    const int st = launch_rms_fwd(r, static_cast<hipStream_t>(stream));
    if (st != PA_OK) return st;
    return finish_launch();
}

int pa_rmsnorm_fwd_many(const pa_rmsnorm* items, int count, void* stream) {
    const int st = launch_rms_fwd_many(items, count, static_cast<hipStream_t>(stream));
    if (st != PA_OK) return st;
    return finish_launch();
}

size_t pa_rmsnorm_bwd_workspace(const pa_rmsnorm* r) {
    if (!r) return 0;
    return rms_bwd_workspace(r);
}

int pa_rmsnorm_bwd(const pa_rmsnorm* r, void* stream) {
    if (!r) return PA_EINVAL;
    const int st = launch_rms_bwd(r, static_cast<hipStream_t>(stream));
    if (st != PA_OK) return st;
    return finish_launch();
}

int pa_linear_small(const pa_linear* l, void* stream) {
    if (!l) return PA_EINVAL;
    const int st = launch_linear_small(l, static_cast<hipStream_t>(stream));
    if (st != PA_OK) return st;
    return finish_launch();
}

}  // extern "C"
