// dn_out_norm: the per-head (gated) RMSNorm after the delta rule
// (OutNorm::forward, src/common/norm.rs:106-144) in one pass: read the
// output row and its gate once, write once.
//
// A head row of head_v_dim values is spread over 16 lanes, CPL = dv / 16
// adjacent values each (two 16-byte loads per lane for bf16 at dv = 256), so
// the mean of squares is four DPP steps inside a 16-lane row; a wave holds 4
// rows, a workgroup 16. Other widths take a generic variant: 64 lanes per
// row, element loads, up to 16 values per lane.
#include <algorithm>
#include <type_traits>

#include "dn_common.hpp"
#include "mfma_util.hpp"

namespace dn {
namespace {

constexpr int kNormThreads = 256;

struct NormParams {
  const void* x;
  const void* gate;
  const float* w;
  void* out;
  int64_t rows;         // tokens·nheads
  int64_t gate_stride;  // elements between tokens' gate rows
  int H, D;
  float eps;
};

template <int LPT>
__device__ inline float lane_group_sum(float x) {
  auto dpp = [](float v, auto ctrl) -> float {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  x += dpp(x, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  x += dpp(x, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  x += dpp(x, std::integral_constant<int, 0x141>{});  // row_half_mirror
  x += dpp(x, std::integral_constant<int, 0x140>{});  // row_mirror: rows of 16
  if constexpr (LPT == 64) {
    x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));  // lane ^ 16
    const float h0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float h1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    x = h0 + h1;
  }
  return x;
}

// CPL values at p: one run of 16-byte vectors (VEC), or element by element
// with channels past the row (i ≥ valid) as 0 and untouched.
template <class T, int N, bool VEC>
__device__ inline void ldn(const T* p, float (&v)[N], int valid) {
  if constexpr (VEC && sizeof(T) == 2 && N % 8 == 0) {
#pragma unroll
    for (int q = 0; q < N / 8; ++q) unpack8(reinterpret_cast<const uint4*>(p)[q], &v[8 * q]);
  } else if constexpr (VEC && sizeof(T) == 4 && N % 4 == 0) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const float4 u = reinterpret_cast<const float4*>(p)[q];
      v[4 * q] = u.x;
      v[4 * q + 1] = u.y;
      v[4 * q + 2] = u.z;
      v[4 * q + 3] = u.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = (!VEC && i >= valid) ? 0.f : ld(p, i);
  }
}

template <class T, int N, bool VEC>
__device__ inline void stn(T* p, const float (&v)[N], int valid) {
  if constexpr (VEC && sizeof(T) == 2 && N % 8 == 0) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int q = 0; q < N / 8; ++q) {
      const u32x4 w = {pk_bf16(v[8 * q], v[8 * q + 1]), pk_bf16(v[8 * q + 2], v[8 * q + 3]),
                       pk_bf16(v[8 * q + 4], v[8 * q + 5]), pk_bf16(v[8 * q + 6], v[8 * q + 7])};
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p) + q);
    }
  } else if constexpr (VEC && sizeof(T) == 4 && N % 4 == 0) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const f32x4 w = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
      __builtin_nontemporal_store(w, reinterpret_cast<f32x4*>(p) + q);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (VEC || i < valid) st(p, i, v[i]);
  }
}

// LPT lanes per row, CPL values per lane. VEC: D == LPT·CPL and aligned rows.
template <class TX, class TG, class TO, int LPT, int CPL, bool VEC, bool GATED>
__global__ __launch_bounds__(kNormThreads) void out_norm_kernel(NormParams p) {
  constexpr int RPB = kNormThreads / LPT;  // rows per workgroup
  const int lane = threadIdx.x % LPT;
  const int64_t row = int64_t(blockIdx.x) * RPB + threadIdx.x / LPT;
  // Rows past the end run on the last row (their lanes take part in no other
  // row's reduction) and store nothing.
  const int64_t rr = row < p.rows ? row : p.rows - 1;
  const int D = p.D, c0 = lane * CPL, valid = D - c0;
  const int64_t t = rr / p.H;
  const int h = int(rr - t * p.H);
  float x[CPL], g[CPL], w[CPL];
  ldn<TX, CPL, VEC>(static_cast<const TX*>(p.x) + rr * D + c0, x, valid);
  if constexpr (GATED)
    ldn<TG, CPL, VEC>(static_cast<const TG*>(p.gate) + t * p.gate_stride + int64_t(h) * D + c0,
                      g, valid);
  ldn<float, CPL, VEC>(p.w + c0, w, valid);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) ss = fmaf(x[i], x[i], ss);
  const float inv = rsqrtf(lane_group_sum<LPT>(ss) / float(D) + p.eps);
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    float y = x[i] * inv * w[i];
    if constexpr (GATED) y *= g[i] * __builtin_amdgcn_rcpf(1.0f + __expf(-g[i]));  // silu
    x[i] = y;
  }
  if (row < p.rows) stn<TO, CPL, VEC>(static_cast<TO*>(p.out) + rr * D + c0, x, valid);
}

template <class TX, class TG, class TO, int LPT, int CPL, bool VEC>
void launch_norm(const NormParams& p, bool gated, hipStream_t stream) {
  constexpr int RPB = kNormThreads / LPT;
  const unsigned grid = unsigned((p.rows + RPB - 1) / RPB);
  if (gated)
    hipLaunchKernelGGL((out_norm_kernel<TX, TG, TO, LPT, CPL, VEC, true>), dim3(grid),
                       dim3(kNormThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((out_norm_kernel<TX, TG, TO, LPT, CPL, VEC, false>), dim3(grid),
                       dim3(kNormThreads), 0, stream, p);
}

template <class TX, class TG, class TO>
hipError_t norm_typed(const NormParams& p, bool gated, bool aligned, hipStream_t stream) {
  const int D = p.D;
  const bool vec = aligned && D % 16 == 0 && (D / 16) * sizeof(TX) % 16 == 0 &&
                   (D / 16) * sizeof(TO) % 16 == 0 && (!gated || (D / 16) * sizeof(TG) % 16 == 0);
  if (vec && D == 256) launch_norm<TX, TG, TO, 16, 16, true>(p, gated, stream);
  else if (vec && D == 128) launch_norm<TX, TG, TO, 16, 8, true>(p, gated, stream);
  else if (D <= 64 * 4) launch_norm<TX, TG, TO, 64, 4, false>(p, gated, stream);
  else launch_norm<TX, TG, TO, 64, 16, false>(p, gated, stream);
  return hipGetLastError();
}

template <class TX, class TG>
hipError_t norm_out(const NormParams& p, int out_dtype, bool gated, bool aligned,
                    hipStream_t stream) {
  return out_dtype == DN_BF16 ? norm_typed<TX, TG, bf16>(p, gated, aligned, stream)
                              : norm_typed<TX, TG, float>(p, gated, aligned, stream);
}

}  // namespace

hipError_t launch_out_norm(const dn_out_norm_args& a, hipStream_t stream) {
  NormParams p{};
  p.x = a.x;
  p.gate = a.gate;
  p.w = a.weight;
  p.out = a.out;
  p.rows = a.tokens * a.nheads;
  p.gate_stride = a.gate_stride;
  p.H = int(a.nheads);
  p.D = int(a.head_v_dim);
  p.eps = float(a.eps);
  const bool gated = a.gate != nullptr;
  auto al = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  const size_t gsz = a.gate_dtype == DN_BF16 ? 2 : 4;
  const bool aligned = al(a.x) && al(a.out) && al(a.weight) &&
                       (!gated || (al(a.gate) && (a.gate_stride * gsz) % 16 == 0));
  ProfScope ps("dn_out_norm", stream);
  const bool xb = a.x_dtype == DN_BF16, gb = a.gate_dtype == DN_BF16;
  if (xb && gb) return norm_out<bf16, bf16>(p, a.out_dtype, gated, aligned, stream);
  if (xb) return norm_out<bf16, float>(p, a.out_dtype, gated, aligned, stream);
  if (gb) return norm_out<float, bf16>(p, a.out_dtype, gated, aligned, stream);
  return norm_out<float, float>(p, a.out_dtype, gated, aligned, stream);
}

}  // namespace dn
