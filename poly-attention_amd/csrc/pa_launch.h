// pa_launch.h -- host-side launchers of the libpolyattn kernels (internal to the library).
#pragma once

#include "pa_common.h"

namespace pa {

// Brackets one kernel launch with HIP events on its stream while pa_profile_start is active
// on this thread (pa_abi.hip); otherwise it costs one thread-local flag test.
struct ProfScope {
    ProfScope(const char* name, hipStream_t s);
    ~ProfScope();
    bool active;
    size_t idx;
    hipStream_t stream;
};

// generic (one lane per row) kernels: every dtype, head dim <= 256, every mask feature
void launch_simt_fwd(const PassDev& P, int dtype, hipStream_t s);
// the epilogue backward: dO (contiguous [B, heads, nq, dim]) and G.droot / G.dgate from the
// gradient of y in G.dout; hr = the root's head count (the pass head count without a root)
void launch_epi_bwd(const GradDev& G, void* dO, int hr, int dtype, hipStream_t s);
// finish the fully-masked rows of an MFMA forward (head dim 64 or 128)
void launch_fwd_fixup(const PassDev& P, int dtype, hipStream_t s);
void launch_simt_bwd(const GradDev& G, int dtype, hipStream_t s, bool pre, bool dq, bool dkv);
// masked passes on the MFMA backward: per-key-head bias-class counts (and, with kterm, the
// key mask folded into a per-key term of row stride nkp), then the fully-masked rows' part
void launch_key_terms(const GradDev& G, float* kterm, int nkp, int32_t* kcnt, int32_t* live,
                      hipStream_t s);
void launch_mask_fixups(const GradDev& G, int dtype, hipStream_t s);

// MFMA kernels (bf16 / f16 / fp32 forward, bf16 / f16 backward; head dim 64 or 128); return
// false when they do not cover P
bool mfma_fwd_f32_supported(const PassDev& P);
void launch_mfma_fwd_f32(const PassDev& P, hipStream_t s);
bool mfma_bwd_f32_supported(const GradDev& G);  // unmasked passes
void launch_mfma_bwd_f32(const GradDev& G, hipStream_t s);
bool mfma_fwd_supported(const PassDev& P, int dtype);
// the short-pass kernel takes this pass (head dim 64, nq, nk <= 64, not causal, no value
// multiplier or key mask, 16-bit)
bool mfma_fwd_short_applies(const PassDev& P, int dtype);
void launch_mfma_fwd(const PassDev& P, int dtype, hipStream_t s);
// both passes of an order-2 chain in one short-pass launch (pass 2's keys / values / key term
// are pass 1's queries / output / lse; the caller checks the views)
bool mfma_order2_short_applies(const PassDev& P1, const PassDev& P2, int dtype);
void launch_order2_short(const PassDev& P1, const PassDev& P2, int dtype, hipStream_t s);
bool mfma_bwd_supported(const GradDev& G, int dtype);
bool mfma_bwd_fuses_pre(const GradDev& G);
void launch_mfma_bwd(const GradDev& G, int dtype, hipStream_t s);

// decode
struct DecodeDev;
size_t decode_workspace_bytes(const pa_decode* d, int* chunk_out, int* nchunks_out);
int launch_decode(const pa_decode* d, hipStream_t s);
// launch_decode on the library's static per-device scratch; *hip_err receives the HIP error
// behind a PA_EHIP
int launch_decode_noalloc(const pa_decode* d, hipStream_t s, int* hip_err);
int launch_prologue(const pa_prologue* p, hipStream_t s);
int launch_rms_fwd(const pa_rmsnorm* p, hipStream_t s);
int launch_rms_fwd_many(const pa_rmsnorm* items, int count, hipStream_t s);
size_t rms_bwd_workspace(const pa_rmsnorm* p);
int launch_rms_bwd(const pa_rmsnorm* p, hipStream_t s);
int launch_linear_small(const pa_linear* l, hipStream_t s);

}  // namespace pa
