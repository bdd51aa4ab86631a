// Shared device/host helpers of the delta-rule core (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstddef>

#include "deltanet_core.h"

namespace dn {

// ---------------------------------------------------------------------------
// bf16 as raw bits: the inputs are plain 16-bit buffers; arithmetic is fp32.
// ---------------------------------------------------------------------------

struct bf16 {
  uint16_t bits;
};

__host__ __device__ inline float bf16_to_f32(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

// Round to nearest even (NaN stays NaN).
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return uint16_t((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// The same rounding in one v_cvt_pk_bf16_f32 (device code).
__device__ inline uint16_t f32_to_bf16_dev(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

template <class T>
__device__ inline float ld(const T* p, size_t i);
template <>
__device__ inline float ld<float>(const float* p, size_t i) {
  return p[i];
}
template <>
__device__ inline float ld<bf16>(const bf16* p, size_t i) {
  return bf16_to_f32(p[i].bits);
}

template <class T>
__device__ inline void st(T* p, size_t i, float v);
template <>
__device__ inline void st<float>(float* p, size_t i, float v) {
  p[i] = v;
}
template <>
__device__ inline void st<bf16>(bf16* p, size_t i, float v) {
  p[i].bits = f32_to_bf16_dev(v);
}

// ---------------------------------------------------------------------------
// Problem dimensions shared by the chunk kernels.
// ---------------------------------------------------------------------------

struct Dims {
  int B, S, H, K, V;
  int ew, ww, dw;  // gate widths; dw = 0 when ungated
  int L, N;        // chunk_len, nchunks = ceil(S / L)
  float scale;
};

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// The MFMA kernels address a chunk's token rows from a per-chunk base with
// 32-bit byte offsets: up to 63 token strides of H·max(K, V) elements, 4
// bytes each for an fp32 y. Shapes whose offsets would wrap take the
// generic kernels (or are refused when MFMA is requested).
inline bool token_rows_fit_32bit(const Dims& d) {
  const int64_t row = int64_t(d.H) * (d.K > d.V ? d.K : d.V);
  return int64_t(4) * 64 * row < (int64_t(1) << 31);
}

// Launch helpers (defined in the per-path translation units).
hipError_t launch_step(const dn_step_args& a, float scale, hipStream_t stream);
// dn_recurrent: the whole sequence in one pass over the state (head_k_dim up
// to kRecMaxK).
constexpr int64_t kRecMaxK = DN_RECURRENT_MAX_K;
bool recurrent_supported(const dn_recurrent_args& a);
hipError_t launch_recurrent(const dn_recurrent_args& a, float scale, hipStream_t stream);
// dn_frontend: the projection front-end (frontend.hip). `parts` selects what
// it writes (launch_frontend: all of it): the q/k units, the v units, the
// write gates, the next conv window (after every read of the old one).
enum FrontParts { kFrontQK = 1, kFrontV = 2, kFrontGates = 4, kFrontWindow = 8, kFrontAll = 15 };
hipError_t launch_frontend(const dn_frontend_args& a, hipStream_t stream, int parts = kFrontAll);
// dn_out_norm: the per-head (gated) RMSNorm (out_norm.hip).
hipError_t launch_out_norm(const dn_out_norm_args& a, hipStream_t stream);
hipError_t launch_unit_lower_inverse(const dn_tri_args& a, hipStream_t stream);
hipError_t launch_block_step(const dn_block_step_args& a, float scale, hipStream_t stream);
int block_step_cols(int64_t head_v_dim);

struct GenericFwdPlan {
  size_t ws_bytes;
};
size_t generic_fwd_workspace(const Dims& d);
hipError_t generic_fwd(const Dims& d, int qkv_dtype, int y_dtype, const void* q, const void* k,
                       const void* v, const float* erase, const float* write, const float* g,
                       const float* state_in, void* y, float* state_out, void* ws,
                       hipStream_t stream);
size_t generic_bwd_workspace(const Dims& d);
hipError_t generic_bwd(const Dims& d, int qkv_dtype, int grad_dtype, const void* dy,
                       const float* dstate_final, const void* q, const void* k, const void* v,
                       const float* erase, const float* write, const float* g,
                       const float* state_in, void* dq, void* dk, void* dv, float* derase,
                       float* dwrite, float* dg, float* dstate, void* ws, hipStream_t stream,
                       void* mfma_ws = nullptr);

bool mfma_fwd_supported(const Dims& d, int qkv_dtype, int y_dtype);
bool mfma_bwd_supported(const Dims& d, int qkv_dtype);
// The MFMA forward: the intra kernel and the scan as two launches with their
// tiles in the workspace, or with `fused` (where fused_fwd_supported holds)
// the one kernel of chunk_fwd_fused.hip.
size_t mfma_fwd_workspace(const Dims& d, bool fused = false);
// The projection front-end's q/k formed in the intra kernel's load stage
// (dn_frontend_chunk_fwd): the raw projection columns, the conv of length 4
// with its window and SiLU (the reference's default activations), the L2
// norm, written to q and k for the scan. Per-head gates, head_k_dim 128,
// bf16 throughout.
struct FeParams {
  const uint16_t* proj;  // [B][S][stride] bf16; q of head h at column h·K, k at (H + h)·K
  long long stride;      // elements between consecutive tokens' rows
  const float* w;        // [conv_dim][4] conv weights (tap j weighs x[t − 3 + j])
  const float* bias;     // [conv_dim] or null
  const uint16_t* win;   // [B][conv_dim][4] bf16, newest column last
  int conv_dim;
  int l2;                // 1: L2 norm over the head (else none)
  uint16_t *q, *k;       // [B][S][H][K] bf16
};
hipError_t mfma_fwd(const Dims& d, int y_dtype, const void* q, const void* k, const void* v,
                    const float* erase, const float* write, const float* g,
                    const float* state_in, void* y, float* state_out, void* ws,
                    hipStream_t stream, bool fused = false, const FeParams* fe = nullptr);
// The MFMA forward with the output norm applied in the scan's y write
// (OutNorm::forward, norm.rs:106-144): y receives the normalised output.
// hipErrorCooperativeLaunchTooLarge, before any launch, when the scan's grid
// cannot be resident at once (its column workgroups exchange sums).
struct FwdNorm {
  const void* gate;       // NULL: OutNorm::Plain; else in y's dtype
  long long gate_stride;  // elements between consecutive tokens' gate rows, below 2^25
  const float* weight;    // γ [V]
  float eps;
  int* fault;             // counts cross-workgroup waits that gave up
  int spin;               // polls before a wait gives up
};
size_t mfma_fwd_norm_workspace(const Dims& d);
// The output-norm scan kernel (chunk_fwd_norm.hip) for head_k_dim K,
// per-channel gates pc, the segmented scan's output pass seg, bf16 y (else
// fp32), `waves`-wave workgroups, gated (else plain) norm.
const void* norm_scan_fn(int K, bool pc, bool seg, bool y_bf16, int waves, bool gated);
hipError_t mfma_fwd_norm(const Dims& d, int y_dtype, const void* q, const void* k, const void* v,
                         const float* erase, const float* write, const float* g,
                         const float* state_in, void* y, float* state_out, void* ws,
                         const FwdNorm& nm, hipStream_t stream);
// The fused forward: per-head gates at head_k_dim 128, head_v_dim a multiple
// of 128, bf16 q/k/v.
bool fused_fwd_supported(const Dims& d, int qkv_dtype);
size_t fused_fwd_workspace(const Dims& d);
hipError_t fused_fwd(const Dims& d, int y_dtype, const void* q, const void* k, const void* v,
                     const float* erase, const float* write, const float* g,
                     const float* state_in, void* y, float* state_out, void* ws,
                     hipStream_t stream);
// The backward's two scans on MFMA (bf16 q/k/v, the shapes mfma_fwd_supported
// accepts): the states entering each chunk and the state cotangents leaving
// each chunk, fp32 [G][K][V], plus the initial state's cotangent. g4: both
// per-chunk arrays in row groups of four instead, [G][K/4][V][4] (a lane's
// four accumulator rows of its column are one 16-byte store), which the
// MFMA chunk-local kernel reads; where states_g4(d) holds, at head_k_dim
// 256 (B=8 T=4096 H=16 dv=256: states scan 2543 → 692 µs, reverse scan
// 3846 → 1623 µs, the chunk-local kernel 5.29 → 5.95 ms, whose key-channel
// phase reads a row as 16-byte-strided words there). At head_k_dim 128 the
// scans gained 80 µs each at dv = 256 and the chunk-local kernel lost 260;
// BASELINE config 5's two-wave scans were slower with it.
size_t mfma_bwd_workspace(const Dims& d);
bool states_g4(const Dims& d);
hipError_t mfma_bwd_scans(const Dims& d, int grad_dtype, const void* dy,
                          const float* dstate_final, const void* q, const void* k, const void* v,
                          const float* erase, const float* write, const float* g,
                          const float* state_in, float* states, float* ds_after, float* dstate,
                          void* ws, hipStream_t stream, bool g4);
// The per-chunk tiles mfma_bwd_scans leaves in its workspace: T (hi, lo) and
// Tᵀ (hi, lo), attnᵀ [G][64][64]; kc = e^{G_last−G}⊙K [G][64][K]; per-channel
// decay: kg = e⊙e^G⊙K hi, lo [G][64][K]; per-head: the cumulative gate [G][64].
struct MfmaTiles {
  const uint16_t *T, *Tlo, *Tt, *Ttl, *AtT, *Kc, *Kg, *Kglo;
  const float* gc;
};
MfmaTiles mfma_bwd_tiles(const Dims& d, void* ws);
// The chunk-local gradients on MFMA (head_v_dim 64, or a multiple of 128 in
// passes of 128 value columns, on top of the shapes of mfma_fwd_supported),
// after mfma_bwd_scans. `partials`: mfma_chunk_bwd_partials(d) bytes of
// workspace for the value-summed gradients between passes.
bool mfma_chunk_bwd_supported(const Dims& d, int qkv_dtype);
size_t mfma_chunk_bwd_partials(const Dims& d);
hipError_t mfma_chunk_bwd(const Dims& d, int grad_dtype, const void* dy, const void* q,
                          const void* k, const void* v, const float* erase, const float* write,
                          const float* g, const float* states, const float* ds_after, void* dq,
                          void* dk, void* dv, float* derase, float* dwrite, float* dg,
                          const MfmaTiles& tiles, float* partials, hipStream_t stream, bool g4);

// Per-kernel HIP-event timing (dn_profile_enable): a scope records a start
// event on construction and a stop event on destruction, on `stream`.
struct ProfScope {
  ProfScope(const char* name, hipStream_t stream);
  ~ProfScope();
  int slot;
  hipStream_t stream;
};

// Compute units of the current device (cached per device; 256 on MI355X).
int device_cu_count();

// Fork / join with the current device's second stream: work launched on
// *side after side_fork(main, side) runs after what `main` already holds and
// may overlap what `main` gets next; side_join(main) makes `main` wait for it.
hipError_t side_fork(hipStream_t main, hipStream_t* side);
hipError_t side_join(hipStream_t main);

// NaN/Inf guard: sets *flag (device int) to 1 if any element is not finite.
hipError_t launch_nonfinite_scan(const void* p, size_t n, int dtype, int* flag,
                                 hipStream_t stream);

}  // namespace dn
