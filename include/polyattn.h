/*
 * polyattn.h -- C ABI of libpolyattn.so, the MI355X (gfx950) poly-attention core.
 *
 * The library computes "attention passes" (one level of the poly-attention chain) and
 * single-token decode steps over the poly KV cache.  It never allocates device memory:
 * every buffer, including scratch workspaces, belongs to the caller.  All calls are
 * asynchronous on the given HIP stream, stateless and re-entrant.
 *
 * Reference interfaces replaced (lucidrains/poly-attention 0.3.6):
 *   pa_attn_pass_fwd   one level of reference_poly_attention / NPolyAttention scores+aggregation
 *                      (poly_attention/poly_attention.py:48-116, n_poly_attention.py:233-313);
 *                      the Triton launch it stands in for is _poly_flash_fwd_kernel
 *                      (flash_poly_attention.py:12-154, launched at :347 and :365); with
 *                      pa_pass.epi also the modules' root-value / gate epilogue
 *                      (poly_attention.py:342-351, n_poly_attention.py:315-326).
 *   pa_poly_order2_fwd both levels of the order-2 chain (poly_attention.py:48-116: the two
 *                      _poly_flash_fwd_kernel launches at flash_poly_attention.py:347 and
 *                      :365), in one launch where both are short passes.
 *   pa_attn_pass_bwd   the backward of one level (flash_poly_attention.py:156-316, launched at
 *                      :409 and :429 inside PolyFlashAttention.backward :386-446).
 *   pa_poly_decode     the cached single-token step of Order2PolyAttention.forward
 *                      (poly_attention.py:283-287, 331-338, 360-363) and of
 *                      NPolyAttention.forward (n_poly_attention.py:196-313, 332-340).
 *   pa_decode_prologue the q norms, rotary embedding and cache appends that precede that
 *                      step (n_poly_attention.py:188-191, 206-207; poly_attention.py:271-276,
 *                      282-286).
 *   pa_rmsnorm_fwd/bwd the per-head q/k RMSNorms of the modules in training and prefill
 *                      (poly_attention.py:271, n_poly_attention.py:188).
 *   pa_linear_small    the nn.Linear projections of a single-token decode step (to_q, to_kvs,
 *                      to_out: poly_attention.py:188-204, n_poly_attention.py:108-120; the
 *                      decode harness's feed-forward and logits, train_enwik8.py:40,148-177)
 *                      when the batch has at most 16 rows.
 *
 * Semantics of one pass (per batch b, pass head h, query row i, key j):
 *   s_ij  = scale * <q[b, h/rq, i], k[b, h/rk, j]>           rq = heads / q.heads, etc.
 *   s_ij  = softclamp * tanh(s_ij / softclamp)              when softclamp > 0
 *   s_ij  = -FLT_MAX  when (causal && j > i) || !key_mask[b, j] || !query_mask[b, i]
 *   s_ij += bias[b, h/rb, j]                                 when bias is given
 *   v_j   = round_to_dtype(v[b, h/rv, j] * vmul[b, h/rm, j]) when vmul is given, else v
 *   out_i = sum_j softmax_j(s_ij) v_j,   lse_i = logsumexp_j(s_ij)   (lse in fp32)
 * The finite -FLT_MAX fill is the reference's (poly_attention.py:68): a row whose entries
 * are all masked is the uniform average over the keys whose score is exactly -FLT_MAX
 * (lse = -FLT_MAX); a row whose entries are all -inf (a masked entry plus a -FLT_MAX
 * bias) yields NaN (lse = -inf), as torch.softmax does.
 */
#ifndef POLYATTN_H
#define POLYATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PA_ABI_VERSION 8
#define PA_MAX_ORDER 8

/* status codes (0 = success, negative = failure) */
#define PA_OK            0
#define PA_EINVAL       -1   /* bad shape, stride, head count or pointer */
#define PA_EUNSUPPORTED -2   /* valid request this build does not implement */
#define PA_EHIP         -3   /* a HIP runtime call failed (pa_last_hip_error) */
#define PA_EWORKSPACE   -4   /* workspace missing or too small */
#define PA_ESCRATCH     -5   /* needs more than the library's static scratch (no-alloc calls) */

/* element types */
#define PA_F32  0
#define PA_F16  1
#define PA_BF16 2

/* pa_pass.flags */
#define PA_FLAG_MAY_DEGENERATE 1   /* masks or -FLT_MAX biases may leave rows fully masked */
#define PA_FLAG_DISCARD_OUT    4   /* pa_poly_order2_fwd, first pass: the caller does not read its
                                      out and lse, which the one-launch path then leaves unwritten
                                      (the buffers are still required) */
/* pa_pass_grad.accumulate bits: add into the gradient buffer instead of overwriting it */
#define PA_ACC_DQ    1
#define PA_ACC_DK    2
#define PA_ACC_DV    4
#define PA_ACC_DVMUL 8
#define PA_ACC_DBIAS 16

/* A strided view of a [batch, heads, n, dim] tensor (or [batch, heads, n] for lse / bias).
 * Strides are in elements; the innermost (dim) stride is 1. ptr == NULL means "absent". */
typedef struct pa_view {
    void*   ptr;
    int64_t sb, sh, sn;
    int32_t heads;   /* head count of this tensor; it divides the pass head count */
    int32_t dtype;   /* PA_F32 / PA_F16 / PA_BF16 */
} pa_view;

/* A [batch, n] keep-mask of bytes (nonzero = keep). ptr == NULL means "no mask". */
typedef struct pa_mask {
    const uint8_t* ptr;
    int64_t sb, sn;
} pa_mask;

/* pa_epilogue.flags */
#define PA_EPI_ROOT_SIGMOID 1   /* the root factor is sigmoid(root) (use_root_value_as_attn_gate) */

/* The modules' epilogue of the final level, applied where the pass stores its output
 * (replaces the element-wise tail of poly_attention.py:342-351 and n_poly_attention.py:
 * 315-326):
 *   y = round(round(r * out) * round(sigmoid(gate))),   r = root, or round(sigmoid(root))
 * with every product and sigmoid rounded to the pass dtype in the order torch evaluates
 * `v2 * out` then `out * gates.sigmoid()`; an absent root or gate drops its factor.  The pass
 * still writes `out` (the backward needs it).  In the backward (pa_pass_grad) `dout` is then
 * the gradient reaching y, and droot / dgate receive the epilogue's input gradients (droot
 * summed over the heads sharing one root head). */
typedef struct pa_epilogue {
    pa_view root;         /* optional [B, hr, nq, dim], dtype of q; hr divides heads */
    pa_view gate;         /* optional [B, heads, nq, dim] */
    pa_view y;            /* [B, heads, nq, dim] */
    int32_t flags;        /* PA_EPI_* */
} pa_epilogue;

/* pa_qk_norm.flags */
#define PA_NORM_Q 1   /* normalise the queries */
#define PA_NORM_K 2   /* normalise the keys */

/* RMSNorms of a pass's queries and / or keys, applied as the kernel loads them instead of by
 * a separate norm kernel (the modules' q norms, poly_attention.py:196-200,271, when nothing
 * else reads the normalised tensors):
 *   x <- round(x * rsqrt(mean(x^2) + eps) * w)
 * with pa_rmsnorm_fwd's arithmetic and summation order (bit-identical results).  Forward
 * only, where the short-pass kernel runs: head dim 64, nq and nk <= 64, not causal, no value
 * multiplier or key mask, bf16 / f16 with weights of the same dtype; PA_EUNSUPPORTED
 * otherwise. */
typedef struct pa_qk_norm {
    const void* q_weight;   /* [dim] with PA_NORM_Q */
    const void* k_weight;   /* [dim] with PA_NORM_K */
    float       q_eps, k_eps;
    int32_t     flags;      /* PA_NORM_* */
} pa_qk_norm;

/* One attention pass (one level of the poly chain). */
typedef struct pa_pass {
    int32_t batch, heads, nq, nk, dim;
    float   scale;        /* usually dim ** -0.5 */
    float   softclamp;    /* <= 0: off */
    int32_t causal;       /* mask j > i (top-left aligned, the reference's triu(1)) */
    int32_t flags;        /* PA_FLAG_* */
    pa_view q, k, v;      /* q: [B, hq, nq, dim]; k, v: [B, hk, nk, dim]; same dtype */
    pa_view vmul;         /* optional element-wise value multiplier, same dtype as v */
    pa_view bias;         /* optional per-key bias [B, hb, nk] (f32, f16 or bf16) */
    pa_mask key_mask;     /* optional [B, nk] */
    pa_mask query_mask;   /* optional [B, nq] */
    pa_view out;          /* [B, heads, nq, dim], dtype of q */
    pa_view lse;          /* [B, heads, nq], PA_F32 */
    const pa_epilogue* epi;  /* optional module epilogue (NULL: none) */
    /* Optional forward workspace of pa_attn_pass_fwd_workspace() bytes (ignored by the
     * backward): with it a key-masked pass folds its key mask into a per-key term and takes
     * the faster forward kernel; without it the results are the same. */
    void*   workspace;
    size_t  workspace_bytes;
    const pa_qk_norm* norm;  /* optional q / k norms on load (NULL: none; forward only) */
} pa_pass;

/* Backward of one pass.  In the backward the key-side tensors (k, v, vmul, bias) must share
 * one head count hk; their gradients are summed over the heads/hk query heads of a group. */
typedef struct pa_pass_grad {
    pa_pass fwd;          /* forward description, with out and lse as written by the forward */
    pa_view dout;         /* [B, heads, nq, dim]; with fwd.epi the gradient of the epilogue's y */
    pa_view dlse;         /* optional fp32 [B, heads, nq]: gradient reaching lse */
    pa_view dq, dk, dv;   /* dq like q; dk, dv like k, v */
    pa_view dvmul;        /* required iff fwd.vmul is given */
    pa_view dbias;        /* optional fp32 [B, hk, nk] */
    int32_t accumulate;   /* PA_ACC_* bits */
    void*   workspace;
    size_t  workspace_bytes;
    pa_view droot;        /* with fwd.epi: required iff it has a root; like root */
    pa_view dgate;        /* with fwd.epi: required iff it has a gate; like gate */
} pa_pass_grad;

/* One level of a cached single-token decode step (see pa_poly_decode). */
typedef struct pa_decode_level {
    pa_view q;            /* [B, hq, 1, dim]: the new token's query for this level */
    pa_view k;            /* [B, kv_heads, n, dim]: keys, the new token at position n-1 */
    pa_view v;            /* [B, hv, n, dim]: values (the msg cache for the final level) */
    pa_view vmul;         /* middle levels: the msg cache of the deeper level */
    pa_view bias;         /* every level but the deepest: the lse cache of the deeper level */
    pa_view out;          /* [B, heads, 1, dim]: the msg cache slot n-1, or the final output */
    pa_view lse;          /* [B, heads, 1]: the lse cache slot n-1 (optional for the final level) */
    int32_t heads;        /* head count of this level (kv_heads or the query head count) */
} pa_decode_level;

/* A single-token decode step of an order-`order` poly attention over a cache of n positions
 * (the new token already written at position n-1 of every q/k/v cache).  levels[0] is the
 * deepest level (scores q_order . q_{order+1}), levels[order-1] the final level (q1 . q2).
 * Level t's value at the new position is: levels[0]: v[n-1]; middle levels:
 * round(v[n-1] * msg_{t-1}); final level: msg_{t-1}, with bias lse_{t-1}, where msg_{t-1}
 * and lse_{t-1} are the step results of level t-1 (also written to its out/lse slots). */
typedef struct pa_decode {
    int32_t batch, kv_heads, n, dim, order;
    float   scale, softclamp;
    int32_t chunk;        /* keys per split-K chunk, 0 = automatic */
    pa_decode_level levels[PA_MAX_ORDER];
    void*   workspace;
    size_t  workspace_bytes;
    /* Optional (NULL = off): a device int32 holding the step's n, for decode loops captured
     * into a HIP graph, where n changes between replays.  `n` above is then the capacity
     * every view holds (n_dev[0] is clamped to 1..n; workspace and grid are sized for n),
     * and the out / lse views of every level but the final one are the whole msg / lse
     * caches (position 0 based): the step writes their position n_dev[0]-1. */
    const int32_t* n_dev;
} pa_decode;

/* One tensor of the decode prologue: the new token's projection for one q / k / v of a
 * level (pa_decode_prologue). */
typedef struct pa_prologue_item {
    pa_view     src;            /* [B, heads, 1, dim]: the projection (any strides, dim stride 1) */
    const void* norm_weight;    /* [dim] RMSNorm weight, or NULL: no normalisation */
    int32_t     weight_dtype;   /* PA_F32 / PA_F16 / PA_BF16 */
    int32_t     rotate;         /* nonzero: rotate the leading rot_dim features after the norm */
    pa_view     out;            /* optional [B, heads, 1, dim]: the resulting row */
    pa_view     cache;          /* optional [B, heads, capacity, dim]: the row also goes to
                                 * position pos of this cache buffer */
} pa_prologue_item;

/* The per-token prologue of a cached decode step: the q RMSNorms, the rotary embedding and
 * the cache appends of one poly-attention layer in one launch.  Every item's rows are
 *   y = round(x * rsqrt(mean(x^2) + eps) * w)                    (when norm_weight is set)
 *   y = round(y * cos(a) + rotate_half(y) * sin(a)) on [0, rot_dim)  (when rotate is set)
 * with rotate_half pairing features (2i, 2i+1) -> (-y[2i+1], y[2i]) and a = angles[feature],
 * computed in fp32 from the (rounded) norm output, as torch evaluates
 *   RMSNorm(dim_head)(q) and apply_rotary_emb(freqs, q)
 * in n_poly_attention.py:188-191 / poly_attention.py:271-276 (the angles as built at
 * train_enwik8.py:143,160-161).  The cache write replaces the torch.cat appends of
 * n_poly_attention.py:206-207 and poly_attention.py:282-286 for fixed-capacity caches.
 * The position is n_dev[0] - 1 when n_dev is given (the step's position count, the same
 * device counter pa_decode.n_dev reads), else `pos`; rows whose position falls outside
 * [0, capacity) are not written to the cache, and then, when `overflow` is given, the kernel
 * sets overflow[0] = 1 (a full fixed-capacity cache; the caller reads the flag after its
 * loop).  All items share src's dtype. */
typedef struct pa_prologue {
    int32_t        batch, dim, count, capacity;
    float          eps;         /* RMSNorm epsilon */
    const void*    angles;      /* [rot_dim] rotary angles of the new position, or NULL */
    int32_t        angles_dtype;/* PA_F32 / PA_F16 / PA_BF16 */
    int32_t        rot_dim;     /* even, <= dim */
    int32_t        pos;         /* cache position when n_dev is NULL */
    const int32_t* n_dev;       /* device: the step's n (positions after the append), or NULL */
    int32_t*       overflow;    /* device int32 [1] set to 1 when the position is outside
                                 * [0, capacity), or NULL */
    /* Without angles: the angles of a rotary module's own positions (poly_attention.py:302-304,
     * n_poly_attention.py:224-229 through rotary-embedding-torch's get_seq_pos / forward),
     * a[f] = p * inv_freq[f / 2] in fp32 with p = round(round(pos) / interp), both roundings to
     * the items' dtype (the rotated tensor's), pos the position written.  NULL: no such rotary. */
    const float*   inv_freq;    /* [rot_dim / 2] */
    float          interp;      /* interpolate_factor (1: none) */
    pa_prologue_item items[2 * PA_MAX_ORDER];
} pa_prologue;

/* Row RMSNorm over the head dim of a [batch, heads, n, dim] view, forward and backward: the
 * q/k norms of the modules, RMSNorm(dim_head) applied to the per-head projections at
 * poly_attention.py:271 and n_poly_attention.py:188 (torch.nn.RMSNorm semantics:
 * y = x * rsqrt(mean(x^2) + eps) * weight, computed in fp32, rounded once), optionally followed
 * by the rotary embedding those lines apply next (poly_attention.py:275-276,
 * n_poly_attention.py:190-191: y = round(t * cos(a) + rotate_half(t) * sin(a)) on the leading
 * rot_dim features, t the rounded norm output, rotate_half pairing (2i, 2i+1) ->
 * (-t[2i+1], t[2i]), a = angles[position * angles_stride + feature]).
 * Forward: x -> y, rstd.  Backward: dy, x, rstd -> dx and (when dweight is set) the weight
 * gradient summed over all rows in fp32, deterministically (workspace:
 * pa_rmsnorm_bwd_workspace bytes); with angles, dy is the gradient of the rotated output and
 * is first rotated back (rounded to the dtype, as the gradient of t).  dim must be a multiple
 * of 8 (4 for fp32) and <= 512; views need 16-byte aligned rows. */
typedef struct pa_rmsnorm {
    int32_t     batch, heads, n, dim;
    float       eps;
    pa_view     x;              /* input, any strides with unit feature stride */
    const void* weight;         /* [dim] or NULL (no affine weight) */
    int32_t     weight_dtype;   /* PA_F32 / PA_F16 / PA_BF16 */
    pa_view     y;              /* forward output (same dtype as x) */
    float*      rstd;           /* [batch * heads * n] fp32: written by the forward, read by the backward;
                                 * NULL in a forward whose backward never runs (not written) */
    pa_view     dy, dx;         /* backward: upstream gradient and input gradient */
    float*      dweight;        /* backward: [dim] fp32 weight gradient, or NULL */
    void*       workspace;
    size_t      workspace_bytes;
    const void* angles;         /* rotary angles [n positions][angles_stride], or NULL */
    int32_t     angles_dtype;   /* PA_F32 / PA_F16 / PA_BF16 */
    int32_t     rot_dim;        /* even, <= dim */
    int64_t     angles_stride;  /* elements between positions (0: one row for all) */
} pa_rmsnorm;

/* Skinny linear layers for decode steps: up to PA_LINEAR_MAX_OUT projections of one input x
 * of rows <= 16 (the batch of a single-token step) in one launch.  Output o computes, with
 * torch.nn.functional.linear semantics (fp32 accumulation, bias in fp32), rounding to dtype
 * after every step as the separate torch ops would:
 *   y = round(x . w^T + bias);  y = round(gelu(y)) when activation = PA_ACT_GELU (the erf
 *   form, torch.nn.GELU());  y = round(y + residual) when residual is set.
 * w is an nn.Linear weight, [out_features, in_features] rows.  All tensors share dtype;
 * strides are row strides in elements (unit innermost stride).  in_features must be a
 * multiple of 8 (4 for fp32), x and every w 16-byte aligned with row strides of whole
 * 16 bytes, and rows * in_features * element size <= 64 KiB. */
#define PA_LINEAR_MAX_OUT 4
#define PA_ACT_NONE 0
#define PA_ACT_GELU 1
typedef struct pa_linear_out {
    const void* w;              /* [out_features, in_features] */
    int64_t     w_stride;
    int32_t     out_features;
    int32_t     activation;     /* PA_ACT_NONE / PA_ACT_GELU */
    const void* bias;           /* [out_features] or NULL */
    const void* residual;       /* [rows, out_features] or NULL */
    int64_t     residual_stride;
    void*       y;              /* [rows, out_features] */
    int64_t     y_stride;
} pa_linear_out;

typedef struct pa_linear {
    int32_t       rows, in_features;
    int32_t       dtype;        /* PA_F32 / PA_F16 / PA_BF16 */
    int32_t       count;        /* outputs, 1 .. PA_LINEAR_MAX_OUT */
    const void*   x;            /* [rows, in_features] */
    int64_t       x_stride;
    /* optional input steps, applied to x before the products (the residual add and pre-norm
     * of a transformer block):  x := round(x + x_add);  x_sum receives that x;
     * x := round(x * rsqrt(mean(x^2) + norm_eps) * norm_weight) when norm is nonzero
     * (torch.nn.RMSNorm(in_features); norm_weight NULL: no affine weight) */
    const void*   x_add;        /* [rows, in_features] or NULL */
    int64_t       x_add_stride;
    void*         x_sum;        /* [rows, in_features] or NULL */
    int64_t       x_sum_stride;
    int32_t       norm;
    int32_t       norm_dtype;   /* dtype of norm_weight */
    const void*   norm_weight;  /* [in_features] or NULL */
    float         norm_eps;
    pa_linear_out out[PA_LINEAR_MAX_OUT];
} pa_linear;

int         pa_abi_version(void);
const char* pa_strerror(int status);
int         pa_last_hip_error(void);   /* hipError_t of the last PA_EHIP on this thread */
/* sizeof of the ABI structs, for binding checks: 0 pa_view, 1 pa_mask, 2 pa_pass,
 * 3 pa_pass_grad, 4 pa_decode_level, 5 pa_decode, 6 pa_prologue_item, 7 pa_prologue,
 * 8 pa_rmsnorm, 9 pa_linear, 10 pa_linear_out, 11 pa_epilogue, 12 pa_qk_norm; 0 for other
 * values */
size_t      pa_struct_size(int which);

/* Kernel timing (no counterpart in the reference: a measurement facility for benchmarks).
 * Between pa_profile_start and pa_profile_stop every kernel this library launches (from any
 * thread of the process) is bracketed by HIP events on its own stream; pa_profile_stop waits
 * for those events and returns per-kernel launch counts and summed durations. */
typedef struct pa_kernel_time {
    const char* name;      /* static string naming the kernel family */
    int64_t     launches;
    double      total_ms;
} pa_kernel_time;
int pa_profile_start(void);
int pa_profile_stop(pa_kernel_time* out, int capacity, int* count);

/* Shader clock under matrix-core load (no counterpart in the reference: a measurement facility
 * for benchmarks, so that a timing can be told apart from a slower-clocked GPU).  Runs a
 * short kernel of independent MFMA chains on every CU (two waves per SIMD, ~50 us) on
 * `stream`, waits for it, and returns in *ghz the waves' mean shader-cycle count (s_memtime)
 * per 100 MHz reference-clock tick (s_memrealtime) over their run, in GHz.  The probe's
 * counts go through a device array of the library: calls that overlap on one GPU race. */
int pa_measure_clock(double* ghz, void* stream);

int    pa_attn_pass_fwd(const pa_pass* p, void* stream);
size_t pa_attn_pass_fwd_workspace(const pa_pass* p);   /* 0: the forward takes none */
size_t pa_attn_pass_bwd_workspace(const pa_pass_grad* g);
int    pa_attn_pass_bwd(const pa_pass_grad* g, void* stream);

/* The two forward passes of an order-2 chain, in order: `second`'s keys, values and key bias
 * must be `first`'s queries, output and lse (the same views; second->nk == first->nq), else
 * PA_EINVAL.  Where both are short passes of the same heads (head dim 64, nq and nk <= 64, not
 * causal, bf16 / f16, no masks, value multiplier or first-pass bias / epilogue, both
 * softclamped or neither; with norms on load, second's key norm the same weight and eps as
 * first's query norm) one kernel runs both: the first pass's output and lse reach the second
 * through on-chip memory (they are still written), and every result has the bits of the two
 * pa_attn_pass_fwd calls it replaces.  Otherwise it makes those two calls. */
int    pa_poly_order2_fwd(const pa_pass* first, const pa_pass* second, void* stream);
size_t pa_poly_decode_workspace(const pa_decode* d);
int    pa_poly_decode(const pa_decode* d, void* stream);

/* pa_poly_decode without a caller workspace.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  The split-K partial records go to a device array
 * of the library instead of d->workspace (ignored, as workspace_bytes): PA_DECODE_SCRATCH_BYTES
 * per GPU, each GPU holding its own copy until the process ends.  A request whose
 * pa_poly_decode_workspace exceeds it returns PA_ESCRATCH without launching.  The call makes
 * no hipMalloc / hipFree or other allocating call; its first call on a device looks the
 * array's device address up once (hipGetSymbolAddress, with that device current).  Every
 * call on one GPU shares that GPU's array and it keeps the last call's contents: each call
 * writes every record it reads before reading it, so nothing has to start at zero, and calls
 * that overlap on one GPU (other streams, other threads) race. */
#define PA_DECODE_SCRATCH_BYTES (16u << 20)
int    pa_poly_decode_noalloc(const pa_decode* d, void* stream);
int    pa_decode_prologue(const pa_prologue* p, void* stream);
int    pa_rmsnorm_fwd(const pa_rmsnorm* r, void* stream);
/* Up to PA_RMS_MAX_ITEMS forwards of one dtype and dim (no rotary angles) in one launch: the
 * q/k norms of a layer (poly_attention.py:271, n_poly_attention.py:188) when no gradient is
 * needed (inference, prefill). */
#define PA_RMS_MAX_ITEMS 4
int    pa_rmsnorm_fwd_many(const pa_rmsnorm* items, int count, void* stream);
size_t pa_rmsnorm_bwd_workspace(const pa_rmsnorm* r);
int    pa_rmsnorm_bwd(const pa_rmsnorm* r, void* stream);
int    pa_linear_small(const pa_linear* l, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* POLYATTN_H */
