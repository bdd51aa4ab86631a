// dn_frontend: the projection front-end between the in-projection GEMM and the
// delta rule (QkvProjection::forward / ::step after in_proj,
// src/common/qkv.rs:373-516) in one pass over the projection.
//
// Work split. A "unit" is one head's channels of one segment: a q head, a k
// head of one micro-step, or a v head. A token's head is spread over LPT = 16
// lanes (32 for heads over 128 channels), CPL = D / LPT adjacent channels
// each, so a wave holds 64 / LPT token rows at once and the L2 norm's sum
// over head_k_dim is a DPP reduction inside one row of lanes. Each lane row
// walks 8 consecutive tokens: it issues all their loads (16-byte vectors for
// bf16 at dk = 128) before any arithmetic, then evaluates the causal
// depthwise convolution (ShortConv, src/common/conv.rs:85-158) from
// registers, newest token first so outputs replace their inputs. The 3 inputs
// before the first token come from the projection, or from the rolling
// window before the sequence starts. The projection is read once from HBM
// (the overlap of neighbouring rows hits in L2) and q, k, v are written once.
// Shapes the vector path does not cover (head widths that are not a multiple
// of LPT, other kernel lengths) take a generic variant: 64 lanes per token,
// element loads, up to 8 taps.
//
// Kernels per call, all HBM-bound byte work: the q, k and v units (one launch
// when head_v_dim is a multiple of head_k_dim, else q + k and v apart), the
// write gates (an elementwise σ with the broadcast layout of squash_write,
// qkv.rs:332-369), and a last small kernel that writes the next rolling
// window once every read of the old one is done, so window_out may alias
// window_in.
#include <algorithm>
#include <type_traits>

#include "activations.hpp"
#include "dn_common.hpp"
#include "mfma_util.hpp"

namespace dn {
namespace {

constexpr int kFrontThreads = 256;  // 4 waves
constexpr int kRowsMaxSeq = 16;     // sequences up to this take frontend_rows_kernel
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct FrontParams {
  const void* proj;
  int64_t stride;      // projection row stride, elements
  const float* w;      // [conv_dim][K]
  const float* bias;   // [conv_dim] or null
  const void* win;     // [B][conv_dim][K]
  int B, S, K;         // K = 0: no convolution
  int conv_dim;        // channels of the convolution (window rows)
  int D;               // head width of this launch's units
  int conv_act;        // applied to the convolution's output
  int win_vec;         // conv length 4 with 16-byte weight rows and aligned windows
  int rows_win;        // the rows kernel writes the next window (one token, win_vec)
  void* wout;          // window_out
  // Up to three unit groups (q, k, v) of head width D in one launch: group g
  // has n[g] units starting at input channel ch0[g], writes nu[g] units per
  // token to out[g], then its activation and norm.
  int n[3];
  int ch0[3];
  int nu[3];
  void* out[3];
  int post_act[3];     // activation after the convolution's (q/k: qk_activation, v: SiLU)
  int norm[3];         // 1: L2 over the head
};

// Sum over each group of LPT lanes (16, 32 or 64), the result in every lane
// of the group: DPP steps inside rows of 16 lanes, then a swizzle across the
// two rows of a 32-lane half, then the halves' sums read back as scalars.
template <int LPT>
__device__ inline float group_sum(float x) {
  auto dpp = [](float v, auto ctrl) -> float {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  x += dpp(x, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]: pairs
  x += dpp(x, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]: quads
  x += dpp(x, std::integral_constant<int, 0x141>{});  // row_half_mirror: groups of 8
  x += dpp(x, std::integral_constant<int, 0x140>{});  // row_mirror: rows of 16
  if constexpr (LPT >= 32)  // lane ^ 16 within each 32-lane half
    x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
  if constexpr (LPT == 64) {
    const float h0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float h1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    x = h0 + h1;
  }
  return x;
}

// N values from p. VEC: one N-wide vector access, no guard (every lane of the
// vector path lies inside its head). Otherwise element by element, channels
// past the head (i ≥ valid) read as 0 and are not touched in memory.
template <class T, int N, bool VEC>
__device__ inline void load_n(const T* p, float (&v)[N], int valid) {
  if constexpr (VEC) {
    (void)valid;
    if constexpr (sizeof(T) == 2) {
      if constexpr (N == 1) {
        v[0] = bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
      } else if constexpr (N == 2) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
        v[0] = __uint_as_float(u << 16);
        v[1] = __uint_as_float(u & 0xffff0000u);
      } else if constexpr (N == 4) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        v[0] = __uint_as_float(u.x << 16);
        v[1] = __uint_as_float(u.x & 0xffff0000u);
        v[2] = __uint_as_float(u.y << 16);
        v[3] = __uint_as_float(u.y & 0xffff0000u);
      } else {
        static_assert(N % 8 == 0, "bf16 vectors of 1, 2, 4 or 8k");
#pragma unroll
        for (int q = 0; q < N / 8; ++q) {
          const uint4 u = reinterpret_cast<const uint4*>(p)[q];
          const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[8 * q + 2 * e] = __uint_as_float(w4[e] << 16);
            v[8 * q + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
          }
        }
      }
    } else {
      if constexpr (N == 1) {
        v[0] = *reinterpret_cast<const float*>(p);
      } else if constexpr (N == 2) {
        const float2 u = *reinterpret_cast<const float2*>(p);
        v[0] = u.x;
        v[1] = u.y;
      } else {
        static_assert(N % 4 == 0, "fp32 vectors of 1, 2 or 4k");
#pragma unroll
        for (int q = 0; q < N / 4; ++q) {
          const float4 u = reinterpret_cast<const float4*>(p)[q];
          v[4 * q] = u.x;
          v[4 * q + 1] = u.y;
          v[4 * q + 2] = u.z;
          v[4 * q + 3] = u.w;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = i < valid ? ld(p, i) : 0.f;
  }
}

template <class T, int N, bool VEC>
__device__ inline void store_n(T* p, const float (&v)[N], int valid) {
  if constexpr (VEC) {
    if constexpr (sizeof(T) == 2) {
      if constexpr (N == 1) {
        *reinterpret_cast<uint16_t*>(p) = f32_to_bf16_dev(v[0]);
      } else {
        uint32_t w[N / 2];
#pragma unroll
        for (int e = 0; e < N / 2; ++e) w[e] = pk_bf16(v[2 * e], v[2 * e + 1]);
        if constexpr (N == 2) {
          *reinterpret_cast<uint32_t*>(p) = w[0];
        } else if constexpr (N == 4) {
          *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
        } else {  // streamed out: non-temporal 16-byte stores
#pragma unroll
          for (int q = 0; q < N / 8; ++q) {
            const u32x4 vv = {w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]};
            __builtin_nontemporal_store(vv, reinterpret_cast<u32x4*>(p) + q);
          }
        }
      }
    } else {
      if constexpr (N == 1) {
        *reinterpret_cast<float*>(p) = v[0];
      } else if constexpr (N == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
      } else {
#pragma unroll
        for (int q = 0; q < N / 4; ++q) {
          const f32x4 vv = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
          __builtin_nontemporal_store(vv, reinterpret_cast<f32x4*>(p) + q);
        }
      }
    }
    (void)valid;
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (i < valid) st(p, i, v[i]);
  }
}

// LPT lanes per token row, CPL channels per lane (LPT·CPL ≥ D), TL tokens per
// lane row. KT register taps: 0 = no convolution; GENERIC = false needs the
// real kernel length K == KT and vector-aligned rows; GENERIC = true takes any
// K ≤ KT (aligned to the newest tap; older taps are skipped) and element
// loads.
// FSILU: the reference's default activations, fixed at compile time (the
// convolution applies SiLU and nothing follows it; qkv.rs:223-229).
template <class TI, class TO, int LPT, int CPL, int TL, int KT, bool GENERIC, bool FSILU>
__global__ __launch_bounds__(kFrontThreads) void frontend_heads_kernel(FrontParams p) {
  constexpr bool VEC = !GENERIC;
  constexpr int R = 64 / LPT;     // token rows per wave
  constexpr int TB = 4 * R * TL;  // tokens per workgroup
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = lane / LPT, l = lane % LPT;
  const int ngrp = (p.S + TB - 1) / TB;
  const int units = p.n[0] + p.n[1] + p.n[2];
  // Units fastest: the resident workgroups cover whole projection rows of
  // consecutive tokens, so the projection streams through HBM row by row.
  const int unit = blockIdx.x % units, rest = blockIdx.x / units;
  const int sg = rest % ngrp, b = rest / ngrp;
  // This lane row's tokens [t0, t0 + TL). Rows past the sequence still run
  // (their lanes take part in no other row's reduction) on clamped indexes
  // and store nothing.
  const int t0 = sg * TB + (wave * R + row) * TL;
  const int g = unit < p.n[0] ? 0 : unit < p.n[0] + p.n[1] ? 1 : 2;
  const int r = unit - (g == 0 ? 0 : g == 1 ? p.n[0] : p.n[0] + p.n[1]);
  const int D = p.D, c0 = l * CPL;
  const int valid = D - c0;  // channels of this lane inside the head (≤ 0: none)
  const int ch = p.ch0[g] + r * D + c0;
  const int S = p.S, K = GENERIC ? p.K : KT;
  const TI* proj = static_cast<const TI*>(p.proj) + size_t(b) * S * p.stride + ch;
  TO* out = static_cast<TO*>(p.out[g]);
  const int post = p.post_act[g], nrm = p.norm[g], nu = p.nu[g];

  // Every token of the lane row in flight at once.
  float xs[TL][CPL];
#pragma unroll
  for (int i = 0; i < TL; ++i)
    load_n<TI, CPL, VEC>(proj + size_t(min(t0 + i, S - 1)) * p.stride, xs[i], valid);
  const bool conv = KT > 0 && K > 0;
  if (conv) {
    constexpr int KP = KT > 1 ? KT - 1 : 1;
    // prev[j] = x[t0 − (KT−1) + j]: the projection (loaded unconditionally at
    // a clamped row, so the loads stay in flight together), then, only in
    // the workgroups that start the sequence, the rolling window before it
    // (window[p + K] holds x[p] for −(K−1) ≤ p < 0), or 0 under a skipped tap.
    float prev[KP][CPL];
#pragma unroll
    for (int j = 0; j < KT - 1; ++j)
      load_n<TI, CPL, VEC>(proj + size_t(min(max(t0 - (KT - 1) + j, 0), S - 1)) * p.stride,
                           prev[j], valid);
    if (sg == 0) {  // workgroup-uniform
#pragma unroll
      for (int j = 0; j < KT - 1; ++j) {
        const int tp = t0 - (KT - 1) + j, wi = tp + K;
#pragma unroll
        for (int i = 0; i < CPL; ++i)
          if (tp < 0)
            prev[j][i] = (wi >= 0 && i < valid)
                             ? ld(static_cast<const TI*>(p.win),
                                  (size_t(b) * p.conv_dim + ch + i) * K + wi)
                             : 0.f;
      }
    }
    // Tap j weighs x[t − (KT−1−j)].
    float wr[KT > 0 ? KT : 1][CPL], bias[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i)
      bias[i] = (p.bias && (!GENERIC || i < valid)) ? p.bias[ch + i] : 0.f;
    if constexpr (!GENERIC && KT == 4) {  // a channel's 4 taps are one 16-byte row
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float4 w4 = *reinterpret_cast<const float4*>(p.w + size_t(ch + i) * 4);
        wr[0][i] = w4.x;
        wr[1][i] = w4.y;
        wr[2][i] = w4.z;
        wr[3][i] = w4.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const int jr = j - (KT - K);  // the real tap, or < 0 for a skipped one
#pragma unroll
        for (int i = 0; i < CPL; ++i)
          wr[j][i] = (jr >= 0 && i < valid) ? p.w[size_t(ch + i) * K + jr] : 0.f;
      }
    }
    // Newest token first, so each output can replace its own input: token n
    // reads inputs n−KT+1 .. n only.
#pragma unroll
    for (int n = TL - 1; n >= 0; --n) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        float y = bias[i];
#pragma unroll
        for (int j = 0; j < KT; ++j) {
          const int src = n - (KT - 1) + j;
          const float xv = src >= 0 ? xs[src >= 0 ? src : 0][i]
                                    : prev[src + KT - 1 >= 0 ? src + KT - 1 : 0][i];
          if constexpr (GENERIC)
            y = j >= KT - K ? fmaf(wr[j][i], xv, y) : y;  // skipped taps are not × 0
          else
            y = fmaf(wr[j][i], xv, y);
        }
        xs[n][i] = FSILU ? y * sigmoidf_(y) : activate(y, p.conv_act);
      }
    }
  }

#pragma unroll
  for (int n = 0; n < TL; ++n) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      if constexpr (GENERIC)
        xs[n][i] = i < valid ? activate(xs[n][i], post) : 0.f;
      else if constexpr (!FSILU)
        xs[n][i] = activate(xs[n][i], post);
      ss = fmaf(xs[n][i], xs[n][i], ss);
    }
    if (nrm) {
      const float inv = rsqrtf(group_sum<LPT>(ss) + 1e-6f);  // norm.rs:83-90
#pragma unroll
      for (int i = 0; i < CPL; ++i) xs[n][i] *= inv;
    }
    if ((!GENERIC || valid > 0) && t0 + n < S)
      store_n<TO, CPL, VEC>(out + (size_t(size_t(b) * S + t0 + n) * nu + r) * D + c0, xs[n],
                            valid);
  }
}

// squash_write (qkv.rs:332-369): σ of the gate columns, the erase part
// doubled under allow_neg_eigval. Output row (b, s) holds the token's u
// micro-steps' gates contiguously, as the raw columns do, so the map is the
// projection row's gate columns [c0, c0 + width) to a dense row of `width`.
struct GateParams {
  const void* proj;
  int64_t stride;
  int64_t rows;        // batch·sequence
  int c0, width;       // raw columns
  float scale;         // 2 under allow_neg_eigval (erase), else 1
  float* out;
  float* out2;         // a second copy (scalar β: erase and write), or null
  int fixed;           // 1: no raw columns, every output is `scale`
};

// One thread per gate value (rows·width < 2³² is checked on the host). The
// grid-stride index is 64-bit: with a 32-bit one, i + stride could wrap past
// 2³² for n close to it and the loop would never end.
template <class TI>
__global__ __launch_bounds__(kFrontThreads) void frontend_gate_kernel(GateParams p) {
  const uint64_t n = uint64_t(p.rows) * uint64_t(p.width);
  for (uint64_t i = uint64_t(blockIdx.x) * kFrontThreads + threadIdx.x; i < n;
       i += uint64_t(gridDim.x) * kFrontThreads) {
    const uint32_t row = uint32_t(i / uint32_t(p.width)), c = uint32_t(i - uint64_t(row) * p.width);
    const float g = p.fixed ? p.scale
                            : p.scale * sigmoidf_(ld(static_cast<const TI*>(p.proj),
                                                     size_t(row) * p.stride + p.c0 + c));
    p.out[i] = g;
    if (p.out2) p.out2[i] = g;
  }
}

// The next rolling window (conv.rs:108-111): the padded input's last K
// columns, padded = [window[1:], x]. One thread per (batch, channel) reads all
// K values before writing any, so window_out may alias window_in.
template <class TI>
__global__ __launch_bounds__(kFrontThreads) void frontend_window_kernel(FrontParams p) {
  const int64_t id = int64_t(blockIdx.x) * kFrontThreads + threadIdx.x;
  if (id >= int64_t(p.B) * p.conv_dim) return;
  const int b = int(id / p.conv_dim), ch = int(id % p.conv_dim);
  const TI* proj = static_cast<const TI*>(p.proj) + size_t(b) * p.S * p.stride + ch;
  const TI* win = static_cast<const TI*>(p.win) + size_t(id) * p.K;
  TI* wout = static_cast<TI*>(p.out[0]) + size_t(id) * p.K;
  float v[DN_FRONTEND_MAX_KERNEL];
#pragma unroll
  for (int j = 0; j < DN_FRONTEND_MAX_KERNEL; ++j) {
    if (j < p.K) {
      const int i = p.S - 1 + j;  // index into padded
      v[j] = i >= p.K - 1 ? ld(proj, size_t(i - (p.K - 1)) * p.stride) : ld(win, 1 + i);
    }
  }
#pragma unroll
  for (int j = 0; j < DN_FRONTEND_MAX_KERNEL; ++j)
    if (j < p.K) st(wout, j, v[j]);
}

// Short sequences (a decode step is one token): a lane row per (batch, token)
// row of one unit instead of per TL tokens of one sequence, so a one-token
// call fills the lanes (the sequence layout leaves 15 of 16 lane rows idle).
// A token's earlier conv inputs come from the projection or, before the
// sequence, from the window, per lane row. Same arithmetic in the same order
// as frontend_heads_kernel. KT = 4: a channel's 4 weights and its window row
// are one vector load each; KT < 0: any conv length up to
// DN_FRONTEND_MAX_KERNEL, element loads; KT = 0: no conv. Vector-aligned rows
// only. WIN (one token per sequence): the lane row also writes the next
// window of its channels, [window[1:], x], from the values it read (no other
// lane reads that row, so window_out may alias window_in).
template <class TI, class TO, int LPT, int CPL, int KT, bool FSILU, bool WIN>
__global__ __launch_bounds__(kFrontThreads) void frontend_rows_kernel(FrontParams p) {
  constexpr int R = 64 / LPT;
  constexpr int RB = 4 * R;  // (batch, token) rows per workgroup
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = lane / LPT, l = lane % LPT;
  const int units = p.n[0] + p.n[1] + p.n[2];
  const int unit = blockIdx.x % units;
  const int64_t nrow = int64_t(p.B) * p.S;
  const int64_t rid = int64_t(blockIdx.x / units) * RB + wave * R + row;
  // Rows past the end run on the last row (their lanes take part in no
  // other row's reduction) and store nothing.
  const int64_t rc = rid < nrow ? rid : nrow - 1;
  const int b = int(rc / p.S), t = int(rc - int64_t(b) * p.S);
  const int g = unit < p.n[0] ? 0 : unit < p.n[0] + p.n[1] ? 1 : 2;
  const int r = unit - (g == 0 ? 0 : g == 1 ? p.n[0] : p.n[0] + p.n[1]);
  const int D = p.D, c0 = l * CPL;
  const int K = KT >= 0 ? KT : p.K;
  const int ch = p.ch0[g] + r * D + c0;
  const TI* proj = static_cast<const TI*>(p.proj) + size_t(b) * p.S * p.stride + ch;
  float x[CPL];
  load_n<TI, CPL, true>(proj + size_t(t) * p.stride, x, CPL);
  if (K > 0) {
    float y[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) y[i] = p.bias ? p.bias[ch + i] : 0.f;
    const size_t wrow = size_t(b) * p.conv_dim + ch;  // window row of channel ch
    if constexpr (KT == 4) {
      // Taps 0..3 weigh x[t−3], x[t−2], x[t−1], x[t].
      float w[CPL][4], xv[CPL][4];
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float4 w4 = *reinterpret_cast<const float4*>(p.w + size_t(ch + i) * 4);
        w[i][0] = w4.x;
        w[i][1] = w4.y;
        w[i][2] = w4.z;
        w[i][3] = w4.w;
      }
      if (t < 3) {  // the window supplies x[t−3 .. −1]: window[tp + 4] holds x[tp]
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
          const TI* wr = static_cast<const TI*>(p.win) + (wrow + i) * 4;
          if constexpr (sizeof(TI) == 2) {
            const uint2 u = *reinterpret_cast<const uint2*>(wr);
            xv[i][0] = __uint_as_float(u.x << 16);
            xv[i][1] = __uint_as_float(u.x & 0xffff0000u);
            xv[i][2] = __uint_as_float(u.y << 16);
            xv[i][3] = __uint_as_float(u.y & 0xffff0000u);
          } else {
            const float4 u = *reinterpret_cast<const float4*>(wr);
            xv[i][0] = u.x;
            xv[i][1] = u.y;
            xv[i][2] = u.z;
            xv[i][3] = u.w;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int tp = t - 3 + j;
        if (tp >= 0) {
          float pv[CPL];
          load_n<TI, CPL, true>(proj + size_t(tp) * p.stride, pv, CPL);
#pragma unroll
          for (int i = 0; i < CPL; ++i) xv[i][j] = pv[i];
        } else {
#pragma unroll
          for (int i = 0; i < CPL; ++i) xv[i][j] = xv[i][tp + 4];
        }
      }
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        xv[i][3] = x[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) y[i] = fmaf(w[i][j], xv[i][j], y[i]);
      }
      if constexpr (WIN) {
        // The next window (one token): the padded input [window[1:], x],
        // which is this token's four taps (bf16 values round-trip exactly).
        // Only real rows write it: a padded row runs on the last real row's
        // channels, and with window_out aliasing window_in it could read that
        // row's window after the real row has replaced it.
#pragma unroll
        for (int i = 0; i < CPL && rid < nrow; ++i) {
          TI* wo = static_cast<TI*>(p.wout) + (wrow + i) * 4;
          if constexpr (sizeof(TI) == 2)
            *reinterpret_cast<uint2*>(wo) = make_uint2(pk_bf16(xv[i][0], xv[i][1]),
                                                       pk_bf16(xv[i][2], xv[i][3]));
          else
            *reinterpret_cast<float4*>(wo) = make_float4(xv[i][0], xv[i][1], xv[i][2], xv[i][3]);
        }
      }
    } else {
      // Tap j weighs x[t − (K−1−j)].
      for (int j = 0; j < K; ++j) {
        const int tp = t - (K - 1 - j);
        float xv[CPL];
        if (tp == t) {
#pragma unroll
          for (int i = 0; i < CPL; ++i) xv[i] = x[i];
        } else if (tp >= 0) {
          load_n<TI, CPL, true>(proj + size_t(tp) * p.stride, xv, CPL);
        } else {  // window[tp + K] holds x[tp] for −(K−1) ≤ tp < 0
#pragma unroll
          for (int i = 0; i < CPL; ++i)
            xv[i] = ld(static_cast<const TI*>(p.win), (wrow + i) * K + tp + K);
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) y[i] = fmaf(p.w[size_t(ch + i) * K + j], xv[i], y[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) x[i] = FSILU ? y[i] * sigmoidf_(y[i]) : activate(y[i], p.conv_act);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    if constexpr (!FSILU) x[i] = activate(x[i], p.post_act[g]);
    ss = fmaf(x[i], x[i], ss);
  }
  if (p.norm[g]) {
    const float inv = rsqrtf(group_sum<LPT>(ss) + 1e-6f);  // norm.rs:83-90
#pragma unroll
    for (int i = 0; i < CPL; ++i) x[i] *= inv;
  }
  if (rid < nrow)
    store_n<TO, CPL, true>(static_cast<TO*>(p.out[g]) + (size_t(rc) * p.nu[g] + r) * D + c0, x,
                           CPL);
}

template <class TI, class TO, int LPT, int CPL, int KT, bool FSILU, bool WIN>
void launch_rows(const FrontParams& p, hipStream_t stream) {
  constexpr int RB = 4 * (64 / LPT);
  const int64_t nblk = (int64_t(p.B) * p.S + RB - 1) / RB;
  const unsigned grid = unsigned(nblk * (p.n[0] + p.n[1] + p.n[2]));
  hipLaunchKernelGGL((frontend_rows_kernel<TI, TO, LPT, CPL, KT, FSILU, WIN>), dim3(grid),
                     dim3(kFrontThreads), 0, stream, p);
}

template <class TI, class TO, int KT, bool FSILU, bool WIN>
void launch_rows_vec(const FrontParams& p, int lpt, int cpl, hipStream_t stream) {
  if (lpt == 32) return launch_rows<TI, TO, 32, 8, KT, FSILU, WIN>(p, stream);  // D = 256
  if (cpl == 8) return launch_rows<TI, TO, 16, 8, KT, FSILU, WIN>(p, stream);
  if (cpl == 4) return launch_rows<TI, TO, 16, 4, KT, FSILU, WIN>(p, stream);
  if (cpl == 2) return launch_rows<TI, TO, 16, 2, KT, FSILU, WIN>(p, stream);
  return launch_rows<TI, TO, 16, 1, KT, FSILU, WIN>(p, stream);
}

template <class TI, class TO, int LPT, int CPL, int TL, int KT, bool GENERIC, bool FSILU = false>
void launch_heads(const FrontParams& p, hipStream_t stream) {
  constexpr int TB = 4 * (64 / LPT) * TL;
  const int ngrp = (p.S + TB - 1) / TB;
  const unsigned grid = unsigned(int64_t(ngrp) * (p.n[0] + p.n[1] + p.n[2]) * p.B);
  hipLaunchKernelGGL((frontend_heads_kernel<TI, TO, LPT, CPL, TL, KT, GENERIC, FSILU>),
                     dim3(grid), dim3(kFrontThreads), 0, stream, p);
}

// The vector path's lanes per token and channels per lane for head width D
// (CPL = D / LPT exactly), or 0 if it has none.
inline int vec_cpl(int D, int* lpt) {
  *lpt = D <= 128 ? 16 : 32;
  if (D % *lpt) return 0;
  const int cpl = D / *lpt;
  return (cpl == 1 || cpl == 2 || cpl == 4 || cpl == 8) ? cpl : 0;
}

template <class TI, class TO, int KT, bool FSILU>
void launch_vec(const FrontParams& p, int lpt, int cpl, hipStream_t stream) {
  if (lpt == 32) return launch_heads<TI, TO, 32, 8, 8, KT, false, FSILU>(p, stream);  // D = 256
  if (cpl == 8) return launch_heads<TI, TO, 16, 8, 8, KT, false, FSILU>(p, stream);
  if (cpl == 4) return launch_heads<TI, TO, 16, 4, 8, KT, false, FSILU>(p, stream);
  if (cpl == 2) return launch_heads<TI, TO, 16, 2, 8, KT, false, FSILU>(p, stream);
  return launch_heads<TI, TO, 16, 1, 8, KT, false, FSILU>(p, stream);
}

// vec_ok: rows, bases and outputs are aligned for the vector path's CPL.
// rows: short sequences take frontend_rows_kernel (needs vec_ok).
template <class TI, class TO>
hipError_t dispatch_heads(const FrontParams& p, bool vec_ok, bool rows, hipStream_t stream) {
  int lpt = 16;
  const int cpl = vec_cpl(p.D, &lpt);
  // The default activations at any conv length (with no conv, none is fused).
  const bool fsilu = p.K > 0 && p.conv_act == DN_ACT_SILU &&
                     (p.n[0] == 0 || p.post_act[0] == DN_ACT_IDENTITY) &&
                     (p.n[1] == 0 || p.post_act[1] == DN_ACT_IDENTITY) &&
                     (p.n[2] == 0 || p.post_act[2] == DN_ACT_IDENTITY);
  if (rows) {
    if (p.K == 0) {
      launch_rows_vec<TI, TO, 0, false, false>(p, lpt, cpl, stream);
    } else if (p.K == 4 && p.win_vec) {
      if (p.rows_win) {
        if (fsilu) launch_rows_vec<TI, TO, 4, true, true>(p, lpt, cpl, stream);
        else launch_rows_vec<TI, TO, 4, false, true>(p, lpt, cpl, stream);
      } else {
        if (fsilu) launch_rows_vec<TI, TO, 4, true, false>(p, lpt, cpl, stream);
        else launch_rows_vec<TI, TO, 4, false, false>(p, lpt, cpl, stream);
      }
    } else {
      if (fsilu) launch_rows_vec<TI, TO, -1, true, false>(p, lpt, cpl, stream);
      else launch_rows_vec<TI, TO, -1, false, false>(p, lpt, cpl, stream);
    }
    return hipGetLastError();
  }
  if (!vec_ok || cpl == 0 || (lpt == 32 && cpl != 8) || (p.K != 0 && p.K != 4)) {
    launch_heads<TI, TO, 64, 4, 4, 8, true>(p, stream);  // any head width ≤ 256, K ≤ 8
  } else if (p.K == 0) {
    launch_vec<TI, TO, 0, false>(p, lpt, cpl, stream);
  } else if (p.conv_act == DN_ACT_SILU &&
             (p.n[0] == 0 || p.post_act[0] == DN_ACT_IDENTITY) &&
             (p.n[1] == 0 || p.post_act[1] == DN_ACT_IDENTITY) &&
             (p.n[2] == 0 || p.post_act[2] == DN_ACT_IDENTITY)) {
    launch_vec<TI, TO, 4, true>(p, lpt, cpl, stream);
  } else {
    launch_vec<TI, TO, 4, false>(p, lpt, cpl, stream);
  }
  return hipGetLastError();
}

template <class TI>
hipError_t launch_gate(const GateParams& g, hipStream_t stream) {
  if (g.width == 0 || g.rows == 0) return hipSuccess;
  const int64_t n = g.rows * g.width;
  const unsigned grid = unsigned(std::min<int64_t>((n + kFrontThreads - 1) / kFrontThreads, 65536));
  hipLaunchKernelGGL(frontend_gate_kernel<TI>, dim3(grid), dim3(kFrontThreads), 0, stream, g);
  return hipGetLastError();
}

template <class TI, class TO>
hipError_t frontend_typed(const dn_frontend_args& a, hipStream_t stream, int parts) {
  const bool do_qk = parts & kFrontQK, do_v = parts & kFrontV;
  const int H = int(a.nheads), dk = int(a.head_k_dim), dv = int(a.head_v_dim);
  const int u = int(a.n_householder), K = int(a.conv_kernel);
  const int key_dim = H * dk, value_dim = H * dv;
  const int conv_dim = key_dim + u * (key_dim + value_dim);
  const bool fused = a.qk_activation == DN_ACT_SILU && K > 0 && a.conv_activation == DN_ACT_SILU;
  const int qk_post = fused ? DN_ACT_IDENTITY : a.qk_activation;
  const int v_post = fused ? DN_ACT_IDENTITY : DN_ACT_SILU;
  const int nrm = a.qk_norm == DN_QKNORM_L2;

  FrontParams p{};
  p.proj = a.projected;
  p.stride = a.proj_stride;
  p.w = a.conv_weight;
  p.bias = a.conv_bias;
  p.win = a.window_in;
  p.B = int(a.batch);
  p.S = int(a.sequence);
  p.K = K;
  p.conv_dim = conv_dim;
  p.conv_act = K > 0 ? a.conv_activation : DN_ACT_IDENTITY;
  auto aligned = [](const void* ptr, size_t bytes) {
    return reinterpret_cast<uintptr_t>(ptr) % bytes == 0;
  };
  // The vector path for head width D: the channel bases of its units and the
  // row stride are multiples of CPL, and the buffers are CPL-vector aligned.
  auto vec_ok = [&](int D, int base_ch, const void* out) {
    int lpt = 16;
    const int cpl = vec_cpl(D, &lpt);
    return cpl > 0 && base_ch % cpl == 0 && a.proj_stride % cpl == 0 &&
           aligned(a.projected, sizeof(TI) * cpl) && aligned(out, sizeof(TO) * cpl);
  };

  ProfScope ps("dn_frontend", stream);
  // q and k: head width head_k_dim, activation and L2 norm.
  p.D = dk;
  p.n[0] = H;
  p.n[1] = u * H;
  p.n[2] = 0;
  p.ch0[0] = 0;
  p.ch0[1] = key_dim;
  p.nu[0] = H;
  p.nu[1] = u * H;
  p.out[0] = a.q;
  p.out[1] = a.k;
  p.post_act[0] = p.post_act[1] = qk_post;
  p.norm[0] = p.norm[1] = nrm;
  const bool qk_vec = vec_ok(dk, 0, a.q) && vec_ok(dk, key_dim, a.k);
  // v: SiLU unless the convolution applied it, no norm. When head_v_dim is a
  // multiple of head_k_dim, a v head is dv/dk units of width dk ([.., H, dv]
  // and [.., H·dv/dk, dk] are the same bytes), and q, k and v share a launch.
  const int vch = key_dim * (1 + u);
  const bool one_launch = qk_vec && dv % dk == 0 && vec_ok(dk, vch, a.v);
  const bool v_vec = one_launch || vec_ok(dv, vch, a.v);
  // Short sequences take the row-per-token kernel wherever the vector path
  // exists; a one-token call with a conv of 4 also writes the next window
  // there, when every unit goes through it.
  auto has_vec = [](int D, bool aligned) {
    int lpt = 16;
    const int cpl = vec_cpl(D, &lpt);
    return aligned && cpl != 0 && !(lpt == 32 && cpl != 8);
  };
  const bool short_seq = p.S <= kRowsMaxSeq;
  const bool rows_qk = short_seq && has_vec(dk, qk_vec);
  const bool rows_v = short_seq && (one_launch ? rows_qk : has_vec(dv, v_vec));
  // Conv length 4 reads a channel's weights and window row as one vector.
  p.win_vec = K == 4 && aligned(a.conv_weight, 16) && aligned(a.window_in, 4 * sizeof(TI)) &&
              aligned(a.window_out, 4 * sizeof(TI));
  p.rows_win = p.S == 1 && p.win_vec && rows_qk && rows_v && do_qk && do_v && (parts & kFrontWindow);
  p.wout = a.window_out;
  hipError_t e = hipSuccess;
  if (!do_qk) p.n[0] = p.n[1] = 0;  // the units of group 2 (v) only, or none
  if (one_launch) {
    p.n[2] = do_v ? u * H * (dv / dk) : 0;
    p.ch0[2] = vch;
    p.nu[2] = u * H * (dv / dk);
    p.out[2] = a.v;
    p.post_act[2] = v_post;
    p.norm[2] = 0;
    if (p.n[0] + p.n[1] + p.n[2] > 0) e = dispatch_heads<TI, TO>(p, true, rows_qk, stream);
  } else {
    if (do_qk) e = dispatch_heads<TI, TO>(p, qk_vec, rows_qk, stream);
    if (e != hipSuccess) return e;
  }
  if (!one_launch && do_v) {
    p.D = dv;
    p.n[0] = u * H;
    p.n[1] = p.n[2] = 0;
    p.ch0[0] = vch;
    p.nu[0] = u * H;
    p.out[0] = a.v;
    p.out[1] = p.out[2] = nullptr;
    p.post_act[0] = v_post;
    p.norm[0] = 0;
    e = dispatch_heads<TI, TO>(p, v_vec, rows_v, stream);
  }
  if (e != hipSuccess) return e;
  // Write gates.
  if (parts & kFrontGates) {
    const float es = a.allow_neg_eigval ? 2.f : 1.f;
    GateParams g{};
    g.proj = a.projected;
    g.stride = a.proj_stride;
    g.rows = a.batch * a.sequence;
    if (a.write_gate == DN_WRITE_FIXED) {
      g.c0 = 0;
      g.width = u * H;
      g.scale = es;
      g.fixed = 1;
      g.out = a.erase;
      g.out2 = a.write == a.erase ? nullptr : a.write;
      e = launch_gate<TI>(g, stream);
    } else if (a.write_gate == DN_WRITE_SCALAR) {
      g.c0 = conv_dim;
      g.width = u * H;
      g.scale = es;
      g.out = a.erase;
      g.out2 = a.write == a.erase ? nullptr : a.write;
      e = launch_gate<TI>(g, stream);
    } else {
      g.c0 = conv_dim;
      g.width = u * key_dim;
      g.scale = es;
      g.out = a.erase;
      e = launch_gate<TI>(g, stream);
      if (e != hipSuccess) return e;
      g.c0 = conv_dim + u * key_dim;
      g.width = u * value_dim;
      g.scale = 1.f;
      g.out = a.write;
      e = launch_gate<TI>(g, stream);
    }
    if (e != hipSuccess) return e;
  }
  // The next window, after every read of the old one above (unless the
  // rows kernel wrote it).
  if ((parts & kFrontWindow) && K > 0 && !p.rows_win) {
    p.out[0] = a.window_out;
    const unsigned grid = unsigned((int64_t(p.B) * conv_dim + kFrontThreads - 1) / kFrontThreads);
    hipLaunchKernelGGL(frontend_window_kernel<TI>, dim3(grid), dim3(kFrontThreads), 0, stream, p);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace

hipError_t launch_frontend(const dn_frontend_args& a, hipStream_t stream, int parts) {
  const bool in_bf = a.in_dtype == DN_BF16, out_bf = a.out_dtype == DN_BF16;
  if (in_bf && out_bf) return frontend_typed<bf16, bf16>(a, stream, parts);
  if (in_bf) return frontend_typed<bf16, float>(a, stream, parts);
  if (out_bf) return frontend_typed<float, bf16>(a, stream, parts);
  return frontend_typed<float, float>(a, stream, parts);
}

}  // namespace dn
