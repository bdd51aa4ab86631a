// dn_block_step: one decode token of a delta-rule block between its in_proj
// and out_proj GEMMs (gated_deltanet_1.rs:218-234) in one launch.
//
// One workgroup of 8 waves per (batch, head) owns the head's whole value row,
// which the output norm reduces over:
//   1. the head's 2·dk + dv convolution channels, one per thread: the short
//      convolution's step (conv.rs:85-158) over the rolling window and the
//      new projection value, the window written back shifted by one, then
//      the convolution's activation and the q/k activation or v's SiLU,
//      evaluated as dn_frontend evaluates them (qkv.rs:454-516);
//   2. the q and k L2 norms (norm.rs:83-90) and kᵀq as three wave sums, then
//      per key row the normalised k, k⊙erase, scale·q and the decay, and per
//      value column v⊙write (squash_write, qkv.rs:332-369);
//   3. delta_step's read-modify-write of the state (recurrent.rs:41-99) laid
//      out as dn_step_row's: a lane owns C = dv/64 consecutive columns of
//      every eighth row, the key-axis sums cross the waves through LDS, and
//      y = S⁻ᵀq' + u·(kᵀq');
//   4. the gated RMSNorm of y over the row (norm.rs:127-134), whose sum of
//      squares is gathered at the step's last barrier.
// The state is loaded first, so its latency covers stages 1 and 2.
#include "activations.hpp"
#include "dn_common.hpp"

namespace dn {
namespace {

constexpr int kBsWaves = 8;
constexpr int kBsThreads = 64 * kBsWaves;

struct BlockParams {
  int H, K, V, KC;
  int conv_dim, key_dim;
  int gate_c0;   // projection column of the first write-gate value
  int norm_c0;   // projection column of the output-norm gate segment, −1 for none
  int64_t stride;
  int conv_act, qk_post, v_post, nrm, write_gate, dw;
  float es, scale, eps;
  const void* proj;
  const float* w;
  const float* bias;
  const void* win;
  void* wout;
  const float* g;
  const float* s_in;
  float* s_out;
  const float* gamma;
  void* out;
  float* y;
};

template <int C>
using vecc = float __attribute__((ext_vector_type(C)));

__device__ inline float wsum64(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <class TI, class TO, int RPT, int C>
__global__ __launch_bounds__(kBsThreads) void block_step_kernel(BlockParams p) {
  constexpr int W = 64 * C;            // columns of the row (≥ dv)
  constexpr int KP = kBsWaves * RPT;   // key rows, zero-padded past dk
  using vec = vecc<C>;
  const int h = blockIdx.x % p.H, b = blockIdx.x / p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int rg = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.K, V = p.V;
  const size_t bh = size_t(b) * p.H + h;
  const int j0 = C * lane;
  const bool colok = j0 < V;  // dv is a multiple of C

  __shared__ float s_k[KP], s_ke[KP], s_q[KP], s_a[KP];
  __shared__ float s_vw[W];
  __shared__ float red_r[kBsWaves][W], red_q[kBsWaves][W];
  __shared__ float s_u[W];
  __shared__ float s_sum[4 + kBsWaves];  // Σq², Σk², kᵀq, —, Σy² of each column wave

  // --- the state, first
  const float* sin = p.s_in + bh * size_t(K) * V + j0;
  vec s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kBsWaves * r;
    s[r] = (i < K && colok)
               ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(sin + size_t(i) * V))
               : vec(0.f);
  }

  // --- 1. the convolution channels: q (dk), k (dk), v (dv) of head h
  const TI* proj = static_cast<const TI*>(p.proj) + size_t(b) * p.stride;
  for (int idx = tid; idx < 2 * K + V; idx += kBsThreads) {
    const int ch = idx < K       ? h * K + idx
                   : idx < 2 * K ? p.key_dim + h * K + (idx - K)
                                 : 2 * p.key_dim + h * V + (idx - 2 * K);
    const float x = ld(proj, ch);
    float yv = x;
    if (p.KC > 0) {
      // The padded input is [window[1:], x]; tap j weighs its j-th column.
      const size_t wrow = (size_t(b) * p.conv_dim + ch) * p.KC;
      const TI* wi = static_cast<const TI*>(p.win) + wrow;
      float tap[DN_FRONTEND_MAX_KERNEL];
#pragma unroll
      for (int j = 0; j < DN_FRONTEND_MAX_KERNEL; ++j)
        tap[j] = j < p.KC - 1 ? ld(wi, j + 1) : x;
      yv = p.bias ? p.bias[ch] : 0.f;
#pragma unroll
      for (int j = 0; j < DN_FRONTEND_MAX_KERNEL; ++j)
        if (j < p.KC) yv = fmaf(p.w[size_t(ch) * p.KC + j], tap[j], yv);
      // The next window: every read of this row is done (window_out may be
      // window_in), and no other thread touches it.
      TI* wo = static_cast<TI*>(p.wout) + wrow;
#pragma unroll
      for (int j = 0; j < DN_FRONTEND_MAX_KERNEL; ++j)
        if (j < p.KC) st(wo, j, tap[j]);
      yv = activate(yv, p.conv_act);
    }
    if (idx < K)
      s_q[idx] = activate(yv, p.qk_post);
    else if (idx < 2 * K)
      s_k[idx - K] = activate(yv, p.qk_post);
    else
      s_vw[idx - 2 * K] = activate(yv, p.v_post);
  }
  for (int i = K + tid; i < KP; i += kBsThreads) s_q[i] = s_k[i] = 0.f;
  for (int j = V + tid; j < W; j += kBsThreads) s_vw[j] = 0.f;
  __syncthreads();

  // --- 2. the norms and kᵀq, then the per-row and per-column coefficients
  if (rg < 3) {
    float acc = 0.f;
    for (int i = lane; i < K; i += 64)
      acc += rg == 0 ? s_q[i] * s_q[i] : rg == 1 ? s_k[i] * s_k[i] : s_k[i] * s_q[i];
    acc = wsum64(acc);
    if (lane == 0) s_sum[rg] = acc;
  }
  __syncthreads();
  const float inv_q = p.nrm ? rsqrtf(s_sum[0] + 1e-6f) : 1.f;
  const float inv_k = p.nrm ? rsqrtf(s_sum[1] + 1e-6f) : 1.f;
  const float kq = s_sum[2] * inv_k * (p.scale * inv_q);
  const float beta = p.write_gate == DN_WRITE_SCALAR ? p.es * sigmoidf_(ld(proj, p.gate_c0 + h))
                                                     : p.es;
  if (tid < KP) {
    const int i = tid, ic = min(i, K - 1);
    const float kk = s_k[i] * inv_k;  // zero past dk
    const float e = p.write_gate == DN_WRITE_CHANNEL
                        ? p.es * sigmoidf_(ld(proj, p.gate_c0 + h * K + ic))
                        : beta;
    s_k[i] = kk;
    s_ke[i] = kk * e;
    s_q[i] = p.scale * (s_q[i] * inv_q);
    s_a[i] = i < K ? (p.dw ? expf(p.g[bh * p.dw + (p.dw == 1 ? 0 : i)]) : 1.0f) : 0.f;
  }
  if (tid < V) {
    const float wv = p.write_gate == DN_WRITE_CHANNEL
                         ? sigmoidf_(ld(proj, p.gate_c0 + p.key_dim + h * V + tid))
                         : beta;
    s_vw[tid] *= wv;
  }
  __syncthreads();

  // --- 3. the delta step
  vec pr = vec(0.f), pq = vec(0.f);
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kBsWaves * r;
    s[r] *= s_a[i];
    pr += s[r] * s_ke[i];
    pq += s[r] * s_q[i];
  }
  *reinterpret_cast<vec*>(&red_r[rg][C * lane]) = pr;
  *reinterpret_cast<vec*>(&red_q[rg][C * lane]) = pq;
  __syncthreads();
  float yv = 0.f;
  if (tid < W) {
    float rr = 0.f, qs = 0.f;
#pragma unroll
    for (int x = 0; x < kBsWaves; ++x) {
      rr += red_r[x][tid];
      qs += red_q[x][tid];
    }
    const float u = s_vw[tid] - rr;
    s_u[tid] = u;
    yv = tid < V ? qs + u * kq : 0.f;
    if (p.y && tid < V) p.y[bh * V + tid] = yv;
  }
  if (rg < W / 64) {
    const float sq = wsum64(yv * yv);
    if (lane == 0) s_sum[4 + rg] = sq;
  }
  __syncthreads();

  // --- 4. the output norm, and the state's write-back
  if (tid < V) {
    float ss = 0.f;
#pragma unroll
    for (int x = 0; x < W / 64; ++x) ss += s_sum[4 + x];
    const float inv = rsqrtf(ss / float(V) + p.eps);
    float o = yv * inv * p.gamma[tid];
    if (p.norm_c0 >= 0) {
      const float z = ld(proj, p.norm_c0 + h * V + tid);
      o *= z * __builtin_amdgcn_rcpf(1.0f + __expf(-z));  // silu
    }
    st(static_cast<TO*>(p.out), bh * V + tid, o);
  }
  const vec uv = *reinterpret_cast<const vec*>(&s_u[C * lane]);
  float* sout = p.s_out + bh * size_t(K) * V + j0;
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kBsWaves * r;
    if (i < K && colok)
      __builtin_nontemporal_store(s[r] + s_k[i] * uv,
                                  reinterpret_cast<vec*>(sout + size_t(i) * V));
  }
}

template <class TI, class TO, int C>
void launch_c(const BlockParams& p, int B, hipStream_t stream) {
  const dim3 grid(unsigned(B * p.H));
#define DN_BS(RPT) \
  hipLaunchKernelGGL((block_step_kernel<TI, TO, RPT, C>), grid, dim3(kBsThreads), 0, stream, p)
  if (p.K <= 64) DN_BS(8);
  else if (p.K <= 128) DN_BS(16);
  else DN_BS(32);
#undef DN_BS
}

template <class TI, class TO>
void launch_typed(const BlockParams& p, int B, int C, hipStream_t stream) {
  if (C == 1) launch_c<TI, TO, 1>(p, B, stream);
  else if (C == 2) launch_c<TI, TO, 2>(p, B, stream);
  else launch_c<TI, TO, 4>(p, B, stream);
}

}  // namespace

// Columns per lane for head_v_dim V: the smallest of 1, 2, 4 with 64·C ≥ V.
int block_step_cols(int64_t V) { return V <= 64 ? 1 : V <= 128 ? 2 : 4; }

hipError_t launch_block_step(const dn_block_step_args& a, float scale, hipStream_t stream) {
  const int H = int(a.nheads), K = int(a.head_k_dim), V = int(a.head_v_dim);
  const int key_dim = H * K, value_dim = H * V;
  const int conv_dim = 2 * key_dim + value_dim;
  const int gate_w = a.write_gate == DN_WRITE_FIXED ? 0
                     : a.write_gate == DN_WRITE_SCALAR ? H
                                                       : key_dim + value_dim;
  const bool has_conv = a.conv_kernel > 0;
  // dn_frontend's activation rule: with the default SiLUs the convolution's
  // SiLU stands for both (qkv.rs:223-229).
  const bool fused = a.qk_activation == DN_ACT_SILU && has_conv && a.conv_activation == DN_ACT_SILU;
  BlockParams p{};
  p.H = H;
  p.K = K;
  p.V = V;
  p.KC = int(a.conv_kernel);
  p.conv_dim = conv_dim;
  p.key_dim = key_dim;
  p.gate_c0 = conv_dim;
  p.norm_c0 = a.norm_gated ? conv_dim + gate_w : -1;
  p.stride = a.proj_stride;
  p.conv_act = has_conv ? a.conv_activation : DN_ACT_IDENTITY;
  p.qk_post = fused ? DN_ACT_IDENTITY : a.qk_activation;
  p.v_post = fused ? DN_ACT_IDENTITY : DN_ACT_SILU;
  p.nrm = a.qk_norm == DN_QKNORM_L2;
  p.write_gate = a.write_gate;
  p.dw = a.has_gate ? int(a.decay_width) : 0;
  p.es = a.allow_neg_eigval ? 2.f : 1.f;
  p.scale = scale;
  p.eps = float(a.eps);
  p.proj = a.projected;
  p.w = a.conv_weight;
  p.bias = a.conv_bias;
  p.win = a.window_in;
  p.wout = a.window_out;
  p.g = a.g;
  p.s_in = a.state_in;
  p.s_out = a.state_out;
  p.gamma = a.norm_weight;
  p.out = a.out;
  p.y = a.y;
  const int C = block_step_cols(V);
  ProfScope ps("dn_block_step", stream);
  const bool in16 = a.in_dtype == DN_BF16, out16 = a.out_dtype == DN_BF16;
  if (in16) {
    if (out16) launch_typed<bf16, bf16>(p, int(a.batch), C, stream);
    else launch_typed<bf16, float>(p, int(a.batch), C, stream);
  } else {
    if (out16) launch_typed<float, bf16>(p, int(a.batch), C, stream);
    else launch_typed<float, float>(p, int(a.batch), C, stream);
  }
  return hipGetLastError();
}

}  // namespace dn
