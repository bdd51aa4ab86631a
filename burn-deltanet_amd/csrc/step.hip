// dn_step: one delta-rule tick (src/delta/recurrent.rs:41-99) as a single
// read-modify-write pass over the fp32 state.
//
// The reference evaluates S⁻ = α⊙S, r = S⁻ᵀ(k⊙erase), u = v⊙write − r,
// S = S⁻ + k uᵀ, y = Sᵀ(scale·q) as separate tensor ops, each a pass over
// [batch, nheads, K, V]. Here both reductions come from one read of S:
//     y = Sᵀq' = S⁻ᵀq' + u (kᵀq'),
// so each element of S is read once and written once — the HBM roofline of
// the step is 2·4·K·V bytes per head plus the token's vectors.
//
// Work split: one workgroup of 256 lanes per (column tile of 64, head, batch).
// Lane t owns columns 4·(t mod 16) … +3 of the tile and rows (t div 16) + 16·r,
// holding its slice of S in registers between the read and the write.

#include "dn_common.hpp"

namespace dn {
namespace {

struct StepParams {
  int B, H, K, V, ew, ww, dw;
  int S;  // tokens (dn_recurrent; 1 for dn_step)
  float scale;
  const void *q, *k, *v;
  const float *erase, *write, *g;
  const float* s_in;
  void* y;
  float* s_out;
};

constexpr int kTileV = 64;
constexpr int kThreads = 256;
constexpr int kRowGroups = kThreads / (kTileV / 4);  // 16

__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <class TQ, class TY, int RPT, bool VEC4>
__global__ __launch_bounds__(kThreads) void step_tile_kernel(StepParams p) {
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int cg = tid & 15, rg = tid >> 4;
  const int K = p.K, V = p.V;
  const int j0 = tile * kTileV + 4 * cg;
  const size_t bh = size_t(b) * p.H + h;

  extern __shared__ float lds[];
  float* s_k = lds;            // k
  float* s_ke = s_k + K;       // k ⊙ erase
  float* s_q = s_ke + K;       // scale · q
  float* s_a = s_q + K;        // exp(g) per key row
  float* red_r = s_a + K;      // [16][64]
  float* red_q = red_r + kRowGroups * kTileV;
  float* s_u = red_q + kRowGroups * kTileV;  // [64]
  float* s_kq = s_u + kTileV;                // [1]

  const TQ* q = static_cast<const TQ*>(p.q) + bh * K;
  const TQ* k = static_cast<const TQ*>(p.k) + bh * K;
  for (int i = tid; i < K; i += kThreads) {
    const float ki = ld(k, i);
    s_k[i] = ki;
    s_ke[i] = ki * p.erase[bh * p.ew + (p.ew == 1 ? 0 : i)];
    s_q[i] = p.scale * ld(q, i);
    s_a[i] = p.dw ? expf(p.g[bh * p.dw + (p.dw == 1 ? 0 : i)]) : 1.0f;
  }
  __syncthreads();
  if (tid < 64) {
    float acc = 0.f;
    for (int i = tid; i < K; i += 64) acc += s_k[i] * s_q[i];
    acc = wave_sum(acc);
    if (tid == 0) s_kq[0] = acc;
  }

  // Read S once; decay it; both partial reductions.
  const float* sin = p.s_in + bh * size_t(K) * V;
  float s[RPT][4];
  float pr[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kRowGroups * r;
    if (i < K) {
      const float* row = sin + size_t(i) * V + j0;
      if (VEC4 && j0 + 3 < V) {
        const float4 x = *reinterpret_cast<const float4*>(row);
        s[r][0] = x.x;
        s[r][1] = x.y;
        s[r][2] = x.z;
        s[r][3] = x.w;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) s[r][c] = (j0 + c < V) ? row[c] : 0.f;
      }
      const float a = s_a[i], ke = s_ke[i], qq = s_q[i];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s[r][c] *= a;
        pr[c] += s[r][c] * ke;
        pq[c] += s[r][c] * qq;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    red_r[rg * kTileV + 4 * cg + c] = pr[c];
    red_q[rg * kTileV + 4 * cg + c] = pq[c];
  }
  __syncthreads();

  // u = v ⊙ write − r;  y = S⁻ᵀq' + u (kᵀq').
  if (tid < kTileV) {
    const int j = tile * kTileV + tid;
    float rr = 0.f, qs = 0.f;
#pragma unroll
    for (int x = 0; x < kRowGroups; ++x) {
      rr += red_r[x * kTileV + tid];
      qs += red_q[x * kTileV + tid];
    }
    float u = 0.f;
    if (j < V) {
      const TQ* v = static_cast<const TQ*>(p.v) + bh * V;
      u = ld(v, j) * p.write[bh * p.ww + (p.ww == 1 ? 0 : j)] - rr;
      st(static_cast<TY*>(p.y), bh * V + j, qs + u * s_kq[0]);
    }
    s_u[tid] = u;
  }
  __syncthreads();

  // S = S⁻ + k uᵀ, written once.
  float* sout = p.s_out + bh * size_t(K) * V;
  float u4[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) u4[c] = s_u[4 * cg + c];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kRowGroups * r;
    if (i < K) {
      const float ki = s_k[i];
      float* row = sout + size_t(i) * V + j0;
      if (VEC4 && j0 + 3 < V) {
        float4 x;
        x.x = s[r][0] + ki * u4[0];
        x.y = s[r][1] + ki * u4[1];
        x.z = s[r][2] + ki * u4[2];
        x.w = s[r][3] + ki * u4[3];
        *reinterpret_cast<float4*>(row) = x;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (j0 + c < V) row[c] = s[r][c] + ki * u4[c];
      }
    }
  }
}

// Row-streaming variant for head_v_dim ≤ 256: a workgroup of 8 waves owns a
// column block of 64·C columns of one (head, batch) and all its K rows; a lane
// owns C consecutive columns, so each wave reads and writes whole 64·C·4-byte
// row segments. The reduction over the key axis crosses the 8 waves through
// LDS. With C = 2 one (head, batch) spans two workgroups of half the
// registers, which doubles the state bytes in flight per CU.
constexpr int kRowWaves = 8;
constexpr int kRowThreads = 64 * kRowWaves;
constexpr int kRowCols = 2;  // columns per lane on the launch path
template <int C>
using ntv = float __attribute__((ext_vector_type(C)));

template <class TQ, class TY, int RPT, int C>
__global__ __launch_bounds__(kRowThreads) void step_row_kernel(StepParams p) {
  constexpr int W = 64 * C;  // columns per workgroup
  using vec = ntv<C>;
  const int nblk = (p.V + W - 1) / W;
  const int cb = blockIdx.x % nblk, bh_id = blockIdx.x / nblk;
  const int h = bh_id % p.H, b = bh_id / p.H;
  const int tid = threadIdx.x, lane = tid & 63, rg = tid >> 6;
  const int K = p.K, V = p.V;
  const int jb = cb * W;       // first column of the block
  const int j0 = jb + C * lane;  // first column of the lane
  const size_t bh = size_t(b) * p.H + h;

  extern __shared__ float lds[];
  float* s_k = lds;
  float* s_ke = s_k + K;
  float* s_q = s_ke + K;
  float* s_a = s_q + K;
  float* red_r = s_a + K;              // [8][W]
  float* red_q = red_r + kRowWaves * W;  // [8][W]
  float* s_u = red_q + kRowWaves * W;    // [W]
  float* s_kq = s_u + W;                 // [1]

  const TQ* q = static_cast<const TQ*>(p.q) + bh * K;
  const TQ* k = static_cast<const TQ*>(p.k) + bh * K;
  for (int i = tid; i < K; i += kRowThreads) {
    const float ki = ld(k, i);
    s_k[i] = ki;
    s_ke[i] = ki * p.erase[bh * p.ew + (p.ew == 1 ? 0 : i)];
    s_q[i] = p.scale * ld(q, i);
    s_a[i] = p.dw ? expf(p.g[bh * p.dw + (p.dw == 1 ? 0 : i)]) : 1.0f;
  }
  __syncthreads();
  if (tid < 64) {
    float acc = 0.f;
    for (int i = tid; i < K; i += 64) acc += s_k[i] * s_q[i];
    acc = wave_sum(acc);
    if (tid == 0) s_kq[0] = acc;
  }

  // The state streams through once per step: non-temporal loads and stores
  // keep it from displacing anything in L2 / Infinity Cache. (Issuing these
  // loads before the gate set-up above measured slower on config 3.)
  const bool colok = j0 + C - 1 < V;
  const float* sin = p.s_in + bh * size_t(K) * V + j0;
  vec s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kRowWaves * r;
    s[r] = (i < K && colok)
               ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(sin + size_t(i) * V))
               : vec(0.f);
  }

  vec pr = vec(0.f), pq = vec(0.f);
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kRowWaves * r;
    if (i < K) {
      s[r] *= s_a[i];
      pr += s[r] * s_ke[i];
      pq += s[r] * s_q[i];
    }
  }
  *reinterpret_cast<vec*>(&red_r[rg * W + C * lane]) = pr;
  *reinterpret_cast<vec*>(&red_q[rg * W + C * lane]) = pq;
  __syncthreads();

  if (tid < W) {
    const int j = jb + tid;
    float rr = 0.f, qs = 0.f;
#pragma unroll
    for (int x = 0; x < kRowWaves; ++x) {
      rr += red_r[x * W + tid];
      qs += red_q[x * W + tid];
    }
    float u = 0.f;
    if (j < V) {
      const TQ* v = static_cast<const TQ*>(p.v) + bh * V;
      u = ld(v, j) * p.write[bh * p.ww + (p.ww == 1 ? 0 : j)] - rr;
      st(static_cast<TY*>(p.y), bh * V + j, qs + u * s_kq[0]);
    }
    s_u[tid] = u;
  }
  __syncthreads();

  const vec uv = *reinterpret_cast<const vec*>(&s_u[C * lane]);
  float* sout = p.s_out + bh * size_t(K) * V + j0;
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kRowWaves * r;
    if (i < K && colok)
      __builtin_nontemporal_store(s[r] + s_k[i] * uv,
                                  reinterpret_cast<vec*>(sout + size_t(i) * V));
  }
}

// dn_recurrent: delta_step over a whole sequence (recurrent.rs:107-142) with
// the state held in registers from the first token to the last, so one call
// reads and writes S once. Same work split as step_row_kernel: a workgroup
// of 8 waves owns 64·C columns of one (head, batch) and all K rows; a lane
// owns C columns of RPT rows. The key-axis reductions cross the waves
// through LDS, two barriers per step. Tokens go two to a step: with α the
// decay, kE = k⊙erase and q' = scale·q of tokens 1 and 2, one pass over S
// gives the columns a = Sᵀ(α₁⊙kE₁), b = Sᵀ(α₁⊙q'₁), c = Sᵀ(α₁α₂⊙kE₂) and
// d = Sᵀ(α₁α₂⊙q'₂), and then, per column,
//   u₁ = vw₁ − a,  y₁ = b + (k₁·q'₁)·u₁,
//   u₂ = vw₂ − c − ((α₂⊙k₁)·kE₂)·u₁,  y₂ = d + ((α₂⊙k₁)·q'₂)·u₁ + (k₂·q'₂)·u₂,
//   S ← α₁α₂⊙S + (α₂⊙k₁)u₁ᵀ + k₂u₂ᵀ,
// the two tokens' delta steps in closed form (the chunkwise WY form at two
// tokens). A DeltaProduct decode token (u = 2 micro-steps) is one step.
//
// Token vectors are staged into LDS TB tokens at a time, every load of a
// block issued before the first LDS write, and the next block is staged
// during the first token of the current one (a short sequence, such as a
// DeltaProduct decode token's micro-steps, is staged whole beside the state
// load). The staged vectors are padded to KP = 8·RPT rows with zeros (decay
// 0 included), so rows past K hold zeros throughout and every LDS read of a
// row is one base register plus an immediate offset.
template <class TQ, class TY, int RPT, int C>
__global__ __launch_bounds__(kRowThreads, RPT <= 16 ? 4 : RPT <= 32 ? 2 : 1) void recurrent_row_kernel(StepParams p) {
  constexpr int W = 64 * C;
  constexpr int KP = kRowWaves * RPT;          // padded rows
  constexpr int TB = 4;                        // tokens per staged block
  constexpr int KI = (TB * KP + kRowThreads - 1) / kRowThreads;  // (token, row) pairs per thread
  constexpr int VI = (TB * W + kRowThreads - 1) / kRowThreads;
  using vec = ntv<C>;
  const int nblk = (p.V + W - 1) / W;
  const int cb = blockIdx.x % nblk, bh_id = blockIdx.x / nblk;
  const int h = bh_id % p.H, b = bh_id / p.H;
  // The wave index is uniform: as a scalar, every row index rg + 8r and the
  // row offsets built on it stay out of the vector registers.
  const int tid = threadIdx.x, lane = tid & 63, rg = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.K, V = p.V, S = p.S;
  const int jb = cb * W, j0 = jb + C * lane;
  const size_t bh = size_t(b) * p.H + h;

  __shared__ float tok[2][TB][4][KP];  // k, k⊙erase, scale·q, α per token
  __shared__ float vw[2][TB][W];       // v⊙write on the block's columns
  __shared__ float red[4][kRowWaves][W];  // per-wave partial sums of a, b, c, d
  __shared__ float s_u[2][W];
  __shared__ float s_dot[4];               // k₁·q'₁, (α₂⊙k₁)·kE₂, (α₂⊙k₁)·q'₂, k₂·q'₂

  const TQ* qp = static_cast<const TQ*>(p.q);
  const TQ* kp = static_cast<const TQ*>(p.k);
  const TQ* vp = static_cast<const TQ*>(p.v);
  // Tokens t0 .. t0+TB−1 into buffer `buf` (inputs laid out [B, S, H, ·]).
  // Indexes past the sequence or the head clamp to its last element, and
  // the values staged for them are zeros (rows) or never read (tokens).
  auto stage = [&](int t0, int buf) {
    float kv[KI], ev[KI], qv[KI], gv[KI], vv[VI], wv[VI];
#pragma unroll
    for (int x = 0; x < KI; ++x) {
      const int idx = min(tid + x * kRowThreads, TB * KP - 1), tt = idx / KP, i = idx % KP;
      const int t = min(t0 + tt, S - 1), ic = min(i, K - 1);
      const size_t row = (size_t(b) * S + t) * p.H + h;
      kv[x] = ld(kp, row * K + ic);
      qv[x] = ld(qp, row * K + ic);
      ev[x] = p.erase[row * p.ew + (p.ew == 1 ? 0 : ic)];
      gv[x] = p.dw ? p.g[row * p.dw + (p.dw == 1 ? 0 : ic)] : 0.f;
    }
#pragma unroll
    for (int x = 0; x < VI; ++x) {
      const int idx = min(tid + x * kRowThreads, TB * W - 1), tt = idx / W;
      const int t = min(t0 + tt, S - 1), jc = min(jb + idx % W, V - 1);
      const size_t row = (size_t(b) * S + t) * p.H + h;
      vv[x] = ld(vp, row * V + jc);
      wv[x] = p.write[row * p.ww + (p.ww == 1 ? 0 : jc)];
    }
#pragma unroll
    for (int x = 0; x < KI; ++x) {
      const int idx = tid + x * kRowThreads, tt = idx / KP, i = idx % KP;
      if (idx < TB * KP) {
        const bool ok = i < K;
        tok[buf][tt][0][i] = ok ? kv[x] : 0.f;
        tok[buf][tt][1][i] = ok ? kv[x] * ev[x] : 0.f;
        tok[buf][tt][2][i] = ok ? p.scale * qv[x] : 0.f;
        tok[buf][tt][3][i] = ok ? (p.dw ? expf(gv[x]) : 1.0f) : 0.f;
      }
    }
#pragma unroll
    for (int x = 0; x < VI; ++x) {
      const int idx = tid + x * kRowThreads;
      if (idx < TB * W) vw[buf][idx / W][idx % W] = jb + idx % W < V ? vv[x] * wv[x] : 0.f;
    }
  };

  const bool colok = j0 + C - 1 < V;
  const float* sin = p.s_in + bh * size_t(K) * V + j0;
  vec s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kRowWaves * r;
    s[r] = (i < K && colok)
               ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(sin + size_t(i) * V))
               : vec(0.f);
  }
  stage(0, 0);
  __syncthreads();
  TY* y = static_cast<TY*>(p.y);
  const int nblocks = (S + TB - 1) / TB;
#pragma unroll 1
  for (int blk = 0; blk < nblocks; ++blk) {
    const int buf = blk & 1, t0 = blk * TB, tn = min(TB, S - t0);
#pragma unroll 1
    for (int tt = 0; tt < tn;) {
      const bool next = tt == 0 && blk + 1 < nblocks;  // stage the next block in this step
      const size_t yrow = ((size_t(b) * S + t0 + tt) * p.H + h) * V + jb + tid;
      if (tt + 1 < tn) {
        // Tokens tt and tt + 1 as one step.
        const float(*d1)[KP] = tok[buf][tt];
        const float(*d2)[KP] = tok[buf][tt + 1];
        // Wave w < 4 forms dot product w over the key axis.
        if (rg < 4) {
          float acc = 0.f;
#pragma unroll
          for (int i = lane; i < KP; i += 64) {
            const float x = rg == 0 ? d1[0][i] : rg == 3 ? d2[0][i] : d1[0][i] * d2[3][i];
            const float z = rg == 0 ? d1[2][i] : rg == 1 ? d2[1][i] : d2[2][i];
            acc += x * z;
          }
          acc = wave_sum(acc);
          if (lane == 0) s_dot[rg] = acc;
        }
        vec pa = vec(0.f), pb = vec(0.f), pc = vec(0.f), pd = vec(0.f);
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
          const int i = rg + kRowWaves * r;
          const float a1 = d1[3][i], a12 = a1 * d2[3][i];
          pa += s[r] * (a1 * d1[1][i]);
          pb += s[r] * (a1 * d1[2][i]);
          pc += s[r] * (a12 * d2[1][i]);
          pd += s[r] * (a12 * d2[2][i]);
          s[r] *= a12;
        }
        *reinterpret_cast<vec*>(&red[0][rg][C * lane]) = pa;
        *reinterpret_cast<vec*>(&red[1][rg][C * lane]) = pb;
        *reinterpret_cast<vec*>(&red[2][rg][C * lane]) = pc;
        *reinterpret_cast<vec*>(&red[3][rg][C * lane]) = pd;
        __syncthreads();
        if (tid < W) {
          float a = 0.f, bq = 0.f, c = 0.f, dq = 0.f;
#pragma unroll
          for (int x = 0; x < kRowWaves; ++x) {
            a += red[0][x][tid];
            bq += red[1][x][tid];
            c += red[2][x][tid];
            dq += red[3][x][tid];
          }
          const float u1 = vw[buf][tt][tid] - a;
          const float u2 = vw[buf][tt + 1][tid] - (c + u1 * s_dot[1]);
          if (jb + tid < V) {
            st(y, yrow, bq + u1 * s_dot[0]);
            st(y, yrow + size_t(p.H) * V, dq + u1 * s_dot[2] + u2 * s_dot[3]);
          }
          s_u[0][tid] = u1;
          s_u[1][tid] = u2;
        }
        if (next) stage(t0 + TB, buf ^ 1);
        __syncthreads();
        const vec u1v = *reinterpret_cast<const vec*>(&s_u[0][C * lane]);
        const vec u2v = *reinterpret_cast<const vec*>(&s_u[1][C * lane]);
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
          const int i = rg + kRowWaves * r;
          s[r] += (d1[0][i] * d2[3][i]) * u1v + d2[0][i] * u2v;
        }
        tt += 2;
      } else {
        // The block's last token alone: S⁻ = α⊙S, u = vw − S⁻ᵀkE,
        // y = S⁻ᵀq' + (k·q')u, S = S⁻ + kuᵀ.
        const float(*d)[KP] = tok[buf][tt];
        if (rg == 0) {
          float acc = 0.f;
#pragma unroll
          for (int i = lane; i < KP; i += 64) acc += d[0][i] * d[2][i];
          acc = wave_sum(acc);
          if (lane == 0) s_dot[0] = acc;
        }
        vec pr = vec(0.f), pq = vec(0.f);
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
          const int i = rg + kRowWaves * r;
          s[r] *= d[3][i];
          pr += s[r] * d[1][i];
          pq += s[r] * d[2][i];
        }
        *reinterpret_cast<vec*>(&red[0][rg][C * lane]) = pr;
        *reinterpret_cast<vec*>(&red[1][rg][C * lane]) = pq;
        __syncthreads();
        if (tid < W) {
          float rr = 0.f, qs = 0.f;
#pragma unroll
          for (int x = 0; x < kRowWaves; ++x) {
            rr += red[0][x][tid];
            qs += red[1][x][tid];
          }
          const float u = vw[buf][tt][tid] - rr;
          if (jb + tid < V) st(y, yrow, qs + u * s_dot[0]);
          s_u[0][tid] = u;
        }
        if (next) stage(t0 + TB, buf ^ 1);
        __syncthreads();
        const vec uv = *reinterpret_cast<const vec*>(&s_u[0][C * lane]);
#pragma unroll
        for (int r = 0; r < RPT; ++r) s[r] += d[0][rg + kRowWaves * r] * uv;
        tt += 1;
      }
    }
  }
  float* sout = p.s_out + bh * size_t(K) * V + j0;
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + kRowWaves * r;
    if (i < K && colok) __builtin_nontemporal_store(s[r], reinterpret_cast<vec*>(sout + size_t(i) * V));
  }
}

template <class TQ, class TY, int C>
hipError_t launch_recurrent_c(const StepParams& p, hipStream_t stream) {
  constexpr int W = 64 * C;
  const dim3 grid(unsigned(p.B * p.H * ((p.V + W - 1) / W)));
  ProfScope ps("dn_recurrent_row", stream);
#define DN_REC(RPT) \
  hipLaunchKernelGGL((recurrent_row_kernel<TQ, TY, RPT, C>), grid, dim3(kRowThreads), 0, stream, p)
  if (p.K <= 64) DN_REC(8);
  else if (p.K <= 128) DN_REC(16);
  else if (p.K <= 256) DN_REC(32);
  else if constexpr (C == 1) DN_REC(64);  // above 256 rows: one column a lane
  else return hipErrorInvalidValue;
#undef DN_REC
  return hipGetLastError();
}

template <class TQ, class TY>
hipError_t launch_recurrent_typed(const StepParams& p, hipStream_t stream) {
  // Two columns per lane (8-byte state accesses) when the rows allow it (up
  // to 256 state rows: 512 would hold 128 registers of state a lane).
  const bool c2 = p.K <= 256 && p.V >= 128 && p.V % 2 == 0 &&
                  ((reinterpret_cast<uintptr_t>(p.s_in) | reinterpret_cast<uintptr_t>(p.s_out)) %
                   8) == 0;
  return c2 ? launch_recurrent_c<TQ, TY, 2>(p, stream) : launch_recurrent_c<TQ, TY, 1>(p, stream);
}

// Fallback for head_k_dim > 512: one workgroup per (head, batch), two passes
// over S (one lane per column).
template <class TQ, class TY>
__global__ __launch_bounds__(kThreads) void step_wide_kernel(StepParams p) {
  const int h = blockIdx.y, b = blockIdx.z;
  const size_t bh = size_t(b) * p.H + h;
  const int K = p.K, V = p.V;
  const TQ* q = static_cast<const TQ*>(p.q) + bh * K;
  const TQ* k = static_cast<const TQ*>(p.k) + bh * K;
  const TQ* v = static_cast<const TQ*>(p.v) + bh * V;
  const float* sin = p.s_in + bh * size_t(K) * V;
  float* sout = p.s_out + bh * size_t(K) * V;
  for (int j = threadIdx.x; j < V; j += kThreads) {
    float rr = 0.f, qs = 0.f, kq = 0.f;
    for (int i = 0; i < K; ++i) {
      const float a = p.dw ? expf(p.g[bh * p.dw + (p.dw == 1 ? 0 : i)]) : 1.0f;
      const float sv = sin[size_t(i) * V + j] * a;
      const float ki = ld(k, i);
      rr += sv * ki * p.erase[bh * p.ew + (p.ew == 1 ? 0 : i)];
      const float qi = p.scale * ld(q, i);
      qs += sv * qi;
      kq += ki * qi;
    }
    const float u = ld(v, j) * p.write[bh * p.ww + (p.ww == 1 ? 0 : j)] - rr;
    st(static_cast<TY*>(p.y), bh * V + j, qs + u * kq);
    for (int i = 0; i < K; ++i) {
      const float a = p.dw ? expf(p.g[bh * p.dw + (p.dw == 1 ? 0 : i)]) : 1.0f;
      sout[size_t(i) * V + j] = sin[size_t(i) * V + j] * a + ld(k, i) * u;
    }
  }
}

template <class TQ, class TY>
hipError_t launch_typed(const StepParams& p, hipStream_t stream) {
  const bool vec4 = (p.V % 4) == 0 &&
                    ((reinterpret_cast<uintptr_t>(p.s_in) | reinterpret_cast<uintptr_t>(p.s_out)) %
                     16) == 0;
  if (vec4 && p.V <= 256 && p.V >= 128 && p.K <= 256) {
    constexpr int W = 64 * kRowCols;
    const size_t lds = sizeof(float) * (4 * size_t(p.K) + 2 * kRowWaves * W + W + 1);
    const dim3 grid(unsigned(p.B * p.H * ((p.V + W - 1) / W)));
    ProfScope ps("dn_step_row", stream);
    if (p.K <= 64)
      hipLaunchKernelGGL((step_row_kernel<TQ, TY, 8, kRowCols>), grid, dim3(kRowThreads), lds,
                         stream, p);
    else if (p.K <= 128)
      hipLaunchKernelGGL((step_row_kernel<TQ, TY, 16, kRowCols>), grid, dim3(kRowThreads), lds,
                         stream, p);
    else
      hipLaunchKernelGGL((step_row_kernel<TQ, TY, 32, kRowCols>), grid, dim3(kRowThreads), lds,
                         stream, p);
    return hipGetLastError();
  }
  const int rpt_needed = (p.K + kRowGroups - 1) / kRowGroups;
  dim3 grid((p.V + kTileV - 1) / kTileV, p.H, p.B);
  const size_t lds = sizeof(float) * (4 * size_t(p.K) + 2 * kRowGroups * kTileV + kTileV + 1);
#define DN_STEP_LAUNCH(RPT)                                                                   \
  do {                                                                                        \
    ProfScope ps("dn_step_tile", stream);                                                     \
    if (vec4)                                                                                 \
      hipLaunchKernelGGL((step_tile_kernel<TQ, TY, RPT, true>), grid, dim3(kThreads), lds,   \
                         stream, p);                                                          \
    else                                                                                      \
      hipLaunchKernelGGL((step_tile_kernel<TQ, TY, RPT, false>), grid, dim3(kThreads), lds,  \
                         stream, p);                                                          \
    return hipGetLastError();                                                                 \
  } while (0)
  if (rpt_needed <= 1) DN_STEP_LAUNCH(1);
  if (rpt_needed <= 2) DN_STEP_LAUNCH(2);
  if (rpt_needed <= 4) DN_STEP_LAUNCH(4);
  if (rpt_needed <= 8) DN_STEP_LAUNCH(8);
  if (rpt_needed <= 16) DN_STEP_LAUNCH(16);
  if (rpt_needed <= 32) DN_STEP_LAUNCH(32);
#undef DN_STEP_LAUNCH
  ProfScope ps("dn_step_wide", stream);
  hipLaunchKernelGGL((step_wide_kernel<TQ, TY>), dim3(1, p.H, p.B), dim3(kThreads), 0, stream,
                     p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_step(const dn_step_args& a, float scale, hipStream_t stream) {
  StepParams p;
  p.S = 1;
  p.B = int(a.batch);
  p.H = int(a.nheads);
  p.K = int(a.head_k_dim);
  p.V = int(a.head_v_dim);
  p.ew = int(a.erase_width);
  p.ww = int(a.write_width);
  p.dw = a.has_gate ? int(a.decay_width) : 0;
  p.scale = scale;
  p.q = a.q;
  p.k = a.k;
  p.v = a.v;
  p.erase = a.erase;
  p.write = a.write;
  p.g = a.g;
  p.s_in = a.state_in;
  p.y = a.y;
  p.s_out = a.state_out;
  const bool qb = a.qkv_dtype == DN_BF16, yb = a.y_dtype == DN_BF16;
  if (qb && yb) return launch_typed<bf16, bf16>(p, stream);
  if (qb) return launch_typed<bf16, float>(p, stream);
  if (yb) return launch_typed<float, bf16>(p, stream);
  return launch_typed<float, float>(p, stream);
}

}  // namespace dn

namespace dn {

bool recurrent_supported(const dn_recurrent_args& a) { return a.head_k_dim <= kRecMaxK; }

hipError_t launch_recurrent(const dn_recurrent_args& a, float scale, hipStream_t stream) {
  StepParams p;
  p.B = int(a.batch);
  p.S = int(a.sequence);
  p.H = int(a.nheads);
  p.K = int(a.head_k_dim);
  p.V = int(a.head_v_dim);
  p.ew = int(a.erase_width);
  p.ww = int(a.write_width);
  p.dw = a.has_gate ? int(a.decay_width) : 0;
  p.scale = scale;
  p.q = a.q;
  p.k = a.k;
  p.v = a.v;
  p.erase = a.erase;
  p.write = a.write;
  p.g = a.g;
  p.s_in = a.state_in;
  p.y = a.y;
  p.s_out = a.state_out;
  const bool qb = a.qkv_dtype == DN_BF16, yb = a.y_dtype == DN_BF16;
  if (qb && yb) return launch_recurrent_typed<bf16, bf16>(p, stream);
  if (qb) return launch_recurrent_typed<bf16, float>(p, stream);
  if (yb) return launch_recurrent_typed<float, bf16>(p, stream);
  return launch_recurrent_typed<float, float>(p, stream);
}

}  // namespace dn
