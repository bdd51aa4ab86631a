// T = (I − N)⁻¹ for a batch of strictly lower triangular N: the standalone
// unit_lower_inverse (src/delta/tri.rs:66-114) with both TriSolve variants.
//
// Blocked (tri.rs:86-98, the default) asks for the exact inverse without
// forming powers of N. Here:
//   size ≤ 64   the chunk kernels' blocked substitution (wy_inverse.hpp) on
//               A = −N padded with zeros to 64: four waves per matrix, each
//               inverting one 16×16 diagonal block by column elimination,
//               then two doubling merges on fp32 MFMA;
//   ≤ 128       one more doubling: the two 64-blocks inverted side by side
//               as above, then T₂₁ = −T₂₂·(A₂₁·T₁₁) on fp32 MFMA;
//   size > 128  forward substitution down 64-column panels: lane j of the
//               panel's wave owns column j and walks its rows in order,
//               t_i = δ_ij + Σ_{j ≤ k < i} N[i][k]·t_k.
// Both read only N's strict lower triangle, as the reference's level masks
// do (tri.rs:116-139).
// Neumann (tri.rs:99-107) sums the series I + N + N² + … + N^{size−1} term by
// term (term ← term·N over the whole matrix, as the reference multiplies it),
// in fp32, so it keeps the series' own rounding where it is ill-conditioned.
#include "dn_common.hpp"
#include "mfma_util.hpp"
#include "wy_inverse.hpp"

namespace dn {
namespace {

__global__ __launch_bounds__(256) void tri_blocked64_kernel(const float* n, float* t, int size) {
  __shared__ float A[kWyL][kWyL + 1];   // −N, strict lower, zero-padded
  __shared__ float Tm[kWyL][kWyL + 1];  // T
  __shared__ float Xs[kWyL / 2][kWyL / 2 + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t base = size_t(blockIdx.x) * size * size;
  for (int idx = tid; idx < kWyL * kWyL; idx += 256) {
    const int i = idx / kWyL, j = idx % kWyL;
    A[i][j] = (j < i && i < size) ? -n[base + size_t(i) * size + j] : 0.f;
    // The merges never write T above its 16×16 block diagonal.
    if (j / 16 > i / 16) Tm[i][j] = 0.f;
  }
  __syncthreads();
  diag_inverse(A, Tm, wave, lane);
  __syncthreads();
  merge_T(A, Tm, Xs, wave, lane, [] { __syncthreads(); });
  for (int idx = tid; idx < size * size; idx += 256) t[base + idx] = Tm[idx / size][idx % size];
}

// 64 < size ≤ 128: T = [[T₁₁, 0], [T₂₁, T₂₂]]. Waves 0-3 invert the first
// 64-block and waves 4-7 the second, each group as tri_blocked64_kernel does
// (the two groups meet the same barriers); then, over the 16 output tiles of
// 16×16, two per wave, P = A₂₁·T₁₁ and T₂₁ = −T₂₂·P (fp32 products; the
// triangular factors' zero blocks are skipped). A₂₁ is read into registers
// at the start and, with P and T₂₁, lives in the diagonal blocks' A once
// the merges are done with it: 75 KB of LDS, two workgroups per CU.
__global__ __launch_bounds__(512) void tri_blocked128_kernel(const float* n, float* t, int size) {
  constexpr int L = kWyL;
  constexpr int NA21 = L * L / 512;  // A₂₁ entries per thread
  __shared__ float A[2][L][L + 1];   // −N's diagonal blocks; then P (A[0]) and A₂₁, T₂₁ (A[1])
  __shared__ float Tm[2][L][L + 1];  // the diagonal blocks' inverses
  __shared__ float Xs[2][L / 2][L / 2 + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave >> 2, w4 = wave & 3, m16 = lane & 15, g4 = lane >> 4;
  const size_t base = size_t(blockIdx.x) * size * size;
  float a21[NA21];
#pragma unroll
  for (int u = 0; u < NA21; ++u) {
    const int idx = tid + 512 * u, i = idx / L, j = idx % L;
    a21[u] = L + i < size ? -n[base + size_t(L + i) * size + j] : 0.f;
  }
  for (int idx = tid; idx < 2 * L * L; idx += 512) {
    const int gb = idx / (L * L), i = (idx / L) % L, j = idx % L;
    const int gi = L * gb + i, gj = L * gb + j;
    A[gb][i][j] = (j < i && gi < size) ? -n[base + size_t(gi) * size + gj] : 0.f;
    if (j / 16 > i / 16) Tm[gb][i][j] = 0.f;
  }
  __syncthreads();
  diag_inverse(A[grp], Tm[grp], w4, lane);
  __syncthreads();
  merge_T(A[grp], Tm[grp], Xs[grp], w4, lane, [] { __syncthreads(); });
  float(*A21)[L + 1] = A[1];
  float(*P)[L + 1] = A[0];
#pragma unroll
  for (int u = 0; u < NA21; ++u) {
    const int idx = tid + 512 * u;
    A21[idx / L][idx % L] = a21[u];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int tt = wave + 8 * u, ti = tt >> 2, tj = tt & 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s4 = 4 * tj; s4 < L / 4; ++s4)  // T₁₁[k][16tj + ·] = 0 for k < 16tj
      acc = mfma_f32(A21[16 * ti + m16][4 * s4 + g4], Tm[0][4 * s4 + g4][16 * tj + m16], acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) P[16 * ti + 4 * g4 + r][16 * tj + m16] = acc[r];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int tt = wave + 8 * u, ti = tt >> 2, tj = tt & 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s4 = 0; s4 < 4 * ti + 4; ++s4)  // T₂₂[16ti + ·][k] = 0 for k ≥ 16ti + 16
      acc = mfma_f32(Tm[1][16 * ti + m16][4 * s4 + g4], P[4 * s4 + g4][16 * tj + m16], acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) A21[16 * ti + 4 * g4 + r][16 * tj + m16] = -acc[r];  // T₂₁
  }
  __syncthreads();
  for (int idx = tid; idx < size * size; idx += 512) {
    const int i = idx / size, j = idx % size;
    const float v = i < L ? (j < L ? Tm[0][i][j] : 0.f)
                          : (j < L ? A21[i - L][j] : Tm[1][i - L][j - L]);
    t[base + idx] = v;
  }
}

// One wave per (matrix, 64-column panel). The panel's columns of T are kept
// in LDS for size ≤ kPanelLds (64 KB), else read back from T itself (each
// lane reads only what it wrote). N's rows are read as wave-uniform values.
constexpr int kPanelLds = 256;

template <bool LDS>
__global__ __launch_bounds__(64) void tri_panel_kernel(const float* n, float* t, int size,
                                                       int npanel) {
  __shared__ float tp[LDS ? kPanelLds * 64 : 1];
  const int lane = threadIdx.x;
  const int panel = blockIdx.x % npanel;
  const size_t base = size_t(blockIdx.x / npanel) * size * size;
  const int j0 = 64 * panel, j = j0 + lane;
  const bool col = j < size;
  float* tcol = t + base + j;  // T[·][j]
  // A lane past the last column reads nothing (its column would run past the
  // matrix); its sums are discarded.
  auto get = [&](int k) {
    if constexpr (LDS) return tp[(k - j0) * 64 + lane];
    return col ? tcol[size_t(k) * size] : 0.f;
  };
  // T is lower triangular: rows above the panel are zero in its columns.
  for (int i = 0; i < j0; ++i)
    if (col) tcol[size_t(i) * size] = 0.f;
  for (int i = j0; i < size; ++i) {
    const float* nrow = n + base + size_t(i) * size;
    float acc = 0.f;
    // t_k = 0 for k < j, so the sum may start at the panel's first column.
    for (int k = j0; k < i; ++k) acc += nrow[k] * get(k);
    const float ti = i == j ? 1.f : (i > j ? acc : 0.f);
    if constexpr (LDS) tp[(i - j0) * 64 + lane] = ti;
    if (col) tcol[size_t(i) * size] = ti;
  }
}

// Neumann: N and the current term in LDS, the running sum in T (each thread
// adds to the entries it owns, tid + 1024·u, so no two threads share one).
template <int MAXN>
__global__ __launch_bounds__(1024) void tri_neumann_kernel(const float* n, float* t, int size) {
  constexpr int P = MAXN + 1;
  constexpr int E = (MAXN * MAXN + 1023) / 1024;
  __shared__ float Ns[MAXN * P], Ts[MAXN * P];
  const int tid = threadIdx.x;
  const int nn = size * size;
  float* tb = t + size_t(blockIdx.x) * nn;
  const float* nb = n + size_t(blockIdx.x) * nn;
  for (int idx = tid; idx < nn; idx += 1024) {
    const int i = idx / size, j = idx % size;
    Ns[i * P + j] = nb[idx];
    Ts[i * P + j] = i == j ? 1.f : 0.f;
    tb[idx] = i == j ? 1.f : 0.f;
  }
  __syncthreads();
  float nxt[E];
  for (int step = 1; step < size; ++step) {
#pragma unroll
    for (int u = 0; u < E; ++u) {
      const int idx = tid + 1024 * u;
      nxt[u] = 0.f;
      if (idx < nn) {
        const int i = idx / size, j = idx % size;
        float s = 0.f;
        for (int k = 0; k < size; ++k) s += Ts[i * P + k] * Ns[k * P + j];
        nxt[u] = s;
      }
    }
    __syncthreads();  // every read of the old term is done
#pragma unroll
    for (int u = 0; u < E; ++u) {
      const int idx = tid + 1024 * u;
      if (idx < nn) {
        Ts[(idx / size) * P + idx % size] = nxt[u];
        tb[idx] += nxt[u];
      }
    }
    __syncthreads();
  }
}

}  // namespace

hipError_t launch_unit_lower_inverse(const dn_tri_args& a, hipStream_t stream) {
  const int size = int(a.size);
  const unsigned batch = unsigned(a.batch);
  if (batch == 0 || size == 0) return hipSuccess;
  if (a.solve == DN_TRI_NEUMANN) {
    ProfScope ps("dn_tri_neumann", stream);
    if (size <= 64)
      hipLaunchKernelGGL(tri_neumann_kernel<64>, dim3(batch), dim3(1024), 0, stream, a.n_strict,
                         a.t, size);
    else
      hipLaunchKernelGGL(tri_neumann_kernel<DN_TRI_NEUMANN_MAX_SIZE>, dim3(batch), dim3(1024), 0,
                         stream, a.n_strict, a.t, size);
  } else if (size <= kWyL) {
    ProfScope ps("dn_tri_blocked64", stream);
    hipLaunchKernelGGL(tri_blocked64_kernel, dim3(batch), dim3(256), 0, stream, a.n_strict, a.t,
                       size);
  } else if (size <= 2 * kWyL) {
    ProfScope ps("dn_tri_blocked128", stream);
    hipLaunchKernelGGL(tri_blocked128_kernel, dim3(batch), dim3(512), 0, stream, a.n_strict, a.t,
                       size);
  } else {
    ProfScope ps("dn_tri_panel", stream);
    const int np = (size + 63) / 64;
    const dim3 grid(unsigned(size_t(batch) * np));
    if (size <= kPanelLds)
      hipLaunchKernelGGL(tri_panel_kernel<true>, grid, dim3(64), 0, stream, a.n_strict, a.t, size,
                         np);
    else
      hipLaunchKernelGGL(tri_panel_kernel<false>, grid, dim3(64), 0, stream, a.n_strict, a.t,
                         size, np);
  }
  return hipGetLastError();
}

}  // namespace dn
