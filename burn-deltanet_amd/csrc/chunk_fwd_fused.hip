// The chunkwise WY forward of per-head gates in one kernel (bf16 MFMA, fp32
// state): Gated DeltaNet / DeltaNet / DeltaProduct at head_k_dim 128, chunk
// 64, erase and write gates of width 1.
//
// The reference runs the chunk forward as prepare → wy (scores, mask, solve,
// U and W) → scan (src/delta/chunk_recalculated/forward.rs:29-440). Here one
// workgroup of eight waves owns (b, h, 128 value columns) for the whole
// sequence and walks its chunks in order. Each wave carries 16 of the
// state's columns in fp32 MFMA accumulators and, beside the scan of chunk n,
// does a share of building chunk n+1's operand tiles in LDS:
//   build (chunk n+1)  stage K, Q and the gates; Akk = e⊙(K Kᵀ)⊙decay and
//                      attn = scale·(Q Kᵀ)⊙decay on MFMA; T = (I + Akk)⁻¹ by
//                      blocked substitution (wy_inverse.hpp); T as bf16 hi +
//                      lo parts, attn, and Kcᵀ = (e^{G_last−G}⊙K)ᵀ
//   scan  (chunk n)    X = w⊙V − (e⊙e^G)⊙(K·S), yᵀ = (scale·e^G)⊙(Sᵀ·Qᵀ),
//                      V' = T·X, yᵀ += V'ᵀ·attnᵀ, S ← e^{G_last}⊙S + Kcᵀ·V'
// so T, attn, Kcᵀ and the cumulative gate never reach HBM: the kernel reads
// q, k, v, the gates and S₀ once and writes y and S once, the path's
// algorithmic bytes (q and k are read by the V/128 workgroups of a head,
// which share an XCD and its L2).
//
// Schedule. The build's dependent steps are spread over the scan's phases,
// six segments per chunk with a workgroup barrier after each:
//   a  Kcᵀ(n)                                ‖ K·S, Sᵀ·Qᵀ, k-steps 0-1
//   b  scores (n+1)                          ‖ k-steps 2-3, X, v (n+1)
//   c  K, Q, gates (n+2) in flight;          ‖ V' = T·X
//      diagonal inverses (n+1)
//   d  merge step 1 (n+1)                    ‖ yᵀ += V'ᵀ·attnᵀ, S += Kcᵀ·V'
//                                              for rows 0-63
//   e  merge steps 2+3 (n+1)                 ‖ rows 64-127, y
//   f  T hi/lo, attn (n+1); gates (n+2)
// The tile buffers are double-buffered by chunk parity, which the loop,
// unrolled by two, knows at compile time. K and Q go from HBM straight into
// LDS (global_load_lds, no registers): chunk n+2's are issued into chunk n's
// slots once segment b has finished reading them, and land before segment b
// of the next chunk reads them. While chunk n+1 is built, its fp32 Akk
// occupies the T slots of its buffer (and the first two rows of the attn
// slot) and T in fp32 the Kcᵀ slot; each is dead before the bf16 tile that
// takes its place is written. attn's blocks above the diagonal are zeroed
// once, then only its first two rows again per chunk.
//
// Layouts. The scan's accumulator tiles serve as MFMA operands in place: an
// operand lane supplies 8 consecutive contraction positions, which a pair of
// vertically adjacent accumulator tiles hold as rows 4q..4q+3 of each. For
// the state S the key channels are therefore assigned to accumulator rows by
// σ (tile rb, row m ↔ channel σ(16·rb + m), σ = perm_pos), which makes a
// lane's 8 state values 8 consecutive channels: K and Q are staged in their
// natural order. X and V' keep tokens in accumulator rows, so T, attn and
// Kcᵀ store their token columns at perm_pos(t), and Kcᵀ its channel rows at
// σ⁻¹(d).

#include <algorithm>
#include <type_traits>

#include "dn_common.hpp"
#include "mfma_util.hpp"
#include "wy_inverse.hpp"

namespace dn {
namespace {

constexpr int kL = kWyL;     // chunk length
constexpr int kW = 8;        // waves per workgroup
constexpr int kT = 64 * kW;  // threads per workgroup
constexpr int kBW = 16 * kW; // value columns per workgroup

struct FusedParams {
  int B, S, H, V, N;
  float scale;
  const uint16_t *q, *k, *v;
  const float *erase, *write, *g;
  const float* s_in;
  void* y;
  float* s_out;
  uint16_t* sink;     // one y row: the target of padded tokens' writes
};

// x, hidden from the optimiser: the build steps derive their lane indices
// from such a copy of the thread id, so that their addresses are recomputed
// inside each step rather than hoisted out of the chunk loop, where they
// would stay live beside the scan's state and spill.
__device__ inline int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// σ⁻¹ of perm_pos (mfma_util.hpp): the row of Kcᵀ that holds key channel d.
__device__ inline int perm_inv(int d) {
  return (d & ~31) + 16 * ((d >> 2) & 1) + 4 * ((d >> 3) & 3) + (d & 3);
}

// One chunk's operand tiles (bf16). K and Q rows are tokens in order, with
// the 16-byte segments of a row XOR-swizzled by the row (tile_at<K>); T, attn
// and Kcᵀ use tile_at<64>.
template <int K>
struct FusedTiles {
  uint16_t Kt[kL * K];
  uint16_t Qt[kL * K];
  uint16_t Th[kL * kL];  // T hi: row i, column perm_pos(j)
  uint16_t Tl[kL * kL];  // T lo
  uint16_t At[kL * kL];  // attn: row i, column perm_pos(j)
  uint16_t Kc[K * kL];   // Kcᵀ: row perm_inv(d), column perm_pos(t)
  uint16_t pad[256];     // T in fp32, built in Kc's place, runs 256 B past it
};

template <int K>
struct FusedShared {
  FusedTiles<K> buf[2];
  // Per-token factors of the chunk in buf[i].
  float gxe[2][kL];   // e·e^G
  float gwr[2][kL];   // w
  float gys[2][kL];   // scale·e^G
  float gex[2][kL];   // e^{G_last − G}
  float gegl[2][4];   // e^{G_last}
  // The chunk whose scores are being formed.
  float gcs[kL];      // in-chunk cumulative gate G
  float ers[kL];      // erase gate
  float xw[4][kL / 2][17];  // the inverse's merge scratch, per wave 0-3
};
static_assert(sizeof(FusedShared<128>) <= 160 * 1024, "one workgroup's LDS");

template <int K, class TY, bool GATED>
__global__ __launch_bounds__(kT) void fused_fwd_kernel(FusedParams p) {
  static_assert(K == 128, "the fused forward is laid out for head_k_dim 128");
  constexpr int KK = K / 32;   // 32-deep k-steps over the key axis
  constexpr int RBK = K / 16;  // 16-row blocks of the state
  constexpr int NLD = kL * K * 2 / 1024 / kW;  // 1 KB runs per wave per K or Q tile
  __shared__ __attribute__((aligned(16))) FusedShared<K> sh;

  const int ntile = p.V / kBW;
  const int BH = p.B * p.H;
  // XCD-aware: the `ntile` workgroups of one (b, h) get ids ≡ (mod 8), so
  // they share an L2 (and q, k reads).
  const int id = blockIdx.x;
  const int group = id / (8 * ntile), within = id % (8 * ntile);
  const int tile = within / 8, bh = group * 8 + within % 8;
  if (bh >= BH) return;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, q4 = lane >> 4, k8 = 8 * q4;
  const size_t tokstride = size_t(p.H);  // rows between consecutive tokens
  const size_t bh_row0 = size_t(b) * p.S * p.H + h;

  // =========================================================================
  // Build: the next chunk's tiles
  // =========================================================================
  // K and Q of chunk c into buffer P, HBM → LDS: each wave moves 1 KB-runs
  // of the swizzled tiles (four rows of 256 B; lane l writes bytes 16l …
  // 16l+15 of its run), the lane's global source being the row segment that
  // the swizzle puts there. Rows past the sequence end read the chunk's last
  // row: their erase and write gates are zero, so they add nothing to A, X,
  // V' or the state, and their y rows go to the sink.
  auto dma_kq = [&](auto P, int c) {
    const int lane = opaque(tid) & 63;
    FusedTiles<K>& T = sh.buf[decltype(P)::value];
    const int tok0 = c * kL;
    const int rl = min(kL, p.S - tok0);  // valid rows (≥ 1)
    const size_t crow = bh_row0 + size_t(tok0) * tokstride;
#pragma unroll
    for (int m = 0; m < NLD; ++m) {
      const int run = wave + kW * m;              // 1 KB run: rows 4·run … 4·run+3
      const int row = 4 * run + (lane >> 4), seg = lane & 15;
      const int c8 = seg ^ (row & 15);            // the logical segment stored there
      const size_t off = (crow + size_t(min(row, rl - 1)) * tokstride) * K + 8 * c8;
      __builtin_amdgcn_global_load_lds(p.k + off,
                                       (__attribute__((address_space(3))) void*)(T.Kt + 512 * run),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds(p.q + off,
                                       (__attribute__((address_space(3))) void*)(T.Qt + 512 * run),
                                       16, 0, 0);
    }
  };
  // The gates of a chunk's tokens, in registers until staged: every wave
  // loads all three for its lane's token (wave 4 uses g and erase, wave 5
  // the write gate), unconditionally and untouched until staged, so nothing
  // waits for them here.
  float gr = 0.f, er = 0.f, wr = 0.f, live = 0.f;
  auto load_gates = [&](int c) {
    const int lane = opaque(tid) & 63;
    const int tok0 = c * kL;
    const int rl = min(kL, p.S - tok0);
    const size_t grow = bh_row0 + size_t(tok0 + min(lane, rl - 1)) * tokstride;
    live = lane < rl ? 1.f : 0.f;  // gates are zero past the end
    gr = GATED ? p.g[grow] : 0.f;
    er = p.erase[grow];
    wr = p.write[grow];
  };
  // Per-token factors of the chunk in buffer P, from the gate registers:
  // waves 4 and 5, which have no share of the inverse's merges.
  auto put_gates = [&](auto P) {
    constexpr int c = decltype(P)::value;
    const int lane = opaque(tid) & 63;
    if (wave == 4) {
      float gv = gr * live;
      const float ev = er * live;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float up = __shfl_up(gv, off, 64);
        if (lane >= off) gv += up;
      }
      const float glast = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), kL - 1));
      const float eg = GATED ? __expf(gv) : 1.f;
      sh.gcs[lane] = gv;
      sh.ers[lane] = ev;
      sh.gex[c][lane] = GATED ? __expf(glast - gv) : 1.f;
      sh.gxe[c][lane] = ev * eg;
      sh.gys[c][lane] = p.scale * eg;
      if (lane == 0) sh.gegl[c][0] = GATED ? __expf(glast) : 1.f;
    } else if (wave == 5) {
      sh.gwr[c][lane] = wr * live;
    }
  };
  // Scratch views of chunk c's buffer while it is built.
  auto Abuf = [&](auto P) {
    return reinterpret_cast<float(*)[kL + 1]>(sh.buf[decltype(P)::value].Th);
  };
  auto Tbuf = [&](auto P) {
    return reinterpret_cast<float(*)[kL + 1]>(sh.buf[decltype(P)::value].Kc);
  };
  // Scores: Akk = e ⊙ (K Kᵀ) ⊙ decay (strict lower) into A, and attn = scale
  // (Q Kᵀ) ⊙ decay kept in registers until its slot is free. The ten lower
  // 16×16 block pairs: wave w takes pair w, waves 6 and 7 also pairs 8, 9.
  uint32_t keep[2][2];  // attn of a pair's four rows, as bf16 pairs
  auto pair_of = [](int pi, int& rb, int& cb) {
    rb = pi < 1 ? 0 : pi < 3 ? 1 : pi < 6 ? 2 : 3;
    cb = pi - rb * (rb + 1) / 2;
  };
  auto scores = [&](auto P) {
    const int lane = opaque(tid) & 63, r16 = lane & 15, q4 = lane >> 4, k8 = 8 * q4;
    FusedTiles<K>& T = sh.buf[decltype(P)::value];
    float(*A)[kL + 1] = Abuf(P);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int pi = s == 0 ? wave : wave + 2;
      if (s == 0 || wave >= 6) {
        int rb, cb;
        pair_of(pi, rb, cb);
        f32x4 acck = {0.f, 0.f, 0.f, 0.f}, accq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const bf16x8 ak = ld8(&T.Kt[tile_at<K>(16 * rb + r16, 32 * kk + k8)]);
          const bf16x8 aq = ld8(&T.Qt[tile_at<K>(16 * rb + r16, 32 * kk + k8)]);
          const bf16x8 bk = ld8(&T.Kt[tile_at<K>(16 * cb + r16, 32 * kk + k8)]);
          acck = mfma16(ak, bk, acck);
          accq = mfma16(aq, bk, accq);
        }
        const int j = 16 * cb + r16, i0 = 16 * rb + 4 * q4;
        const float gj = sh.gcs[j];
        // The lane's four rows i0 … i0+3: G and the erase gate, one read each.
        const float4 g4 = *reinterpret_cast<const float4*>(&sh.gcs[i0]);
        const float4 e4 = *reinterpret_cast<const float4*>(&sh.ers[i0]);
        const float gi[4] = {g4.x, g4.y, g4.z, g4.w}, ei[4] = {e4.x, e4.y, e4.z, e4.w};
        float at[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = i0 + r;
          // G is non-increasing, so the exponent is ≤ 0 wherever it is kept;
          // the clamp keeps the masked (j > i) lanes finite.
          const float e = GATED ? __expf(fminf(gi[r] - gj, 0.f)) : 1.f;
          const float decay = (j <= i) ? e : 0.f;
          const float akk = ei[r] * acck[r] * decay;
          A[i][j] = (j < i) ? akk : 0.f;
          at[r] = p.scale * accq[r] * decay;
        }
        keep[s][0] = pk_bf16(at[0], at[1]);
        keep[s][1] = pk_bf16(at[2], at[3]);
      }
    }
  };
  // Diagonal blocks of T (waves 0-3). T above its block diagonal is neither
  // written nor read in fp32: finish_t writes its zeros.
  auto diag = [&](auto P) {
    const int lane = opaque(threadIdx.x) & 63;
    if (wave < 4) diag_inverse(Abuf(P), Tbuf(P), wave, lane);
  };
  // T hi / lo and attn of chunk c into its buffer (A is dead; T in fp32 is
  // read from the Kc slot). Thread: row tid/8, natural columns 8·(tid%8) …
  // +7 as two groups of four consecutive positions of perm_pos.
  auto finish_t = [&](auto P) {
    const int tid = opaque(threadIdx.x), lane = tid & 63, r16 = lane & 15, q4 = lane >> 4;
    FusedTiles<K>& T = sh.buf[decltype(P)::value];
    const float(*Tm)[kL + 1] = Tbuf(P);
    const int row = tid / 8, c0 = 8 * (tid % 8);
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      const bool upper = (c0 + 4 * gq) / 16 > row / 16;  // a zero block of T
      float tv[4];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) tv[cc] = upper ? 0.f : Tm[row][c0 + 4 * gq + cc];
      const int at = tile_at<kL>(row, perm_pos(c0 + 4 * gq));
      const uint32_t h0 = pk_bf16(tv[0], tv[1]), h1 = pk_bf16(tv[2], tv[3]);
      const uint32_t l0 = pk_bf16(tv[0] - lo_f(h0), tv[1] - hi_f(h0));
      const uint32_t l1 = pk_bf16(tv[2] - lo_f(h1), tv[3] - hi_f(h1));
      *reinterpret_cast<uint2*>(&T.Th[at]) = make_uint2(h0, h1);
      *reinterpret_cast<uint2*>(&T.Tl[at]) = make_uint2(l0, l1);
    }
    // attn from the registers; its zero blocks above the diagonal.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s == 0 || wave >= 6) {
        int rb, cb;
        pair_of(s == 0 ? wave : wave + 2, rb, cb);
        const int pj = perm_pos(16 * cb + r16);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          T.At[tile_at<kL>(16 * rb + 4 * q4 + r, pj)] =
              uint16_t((r & 1) ? keep[s][r >> 1] >> 16 : keep[s][r >> 1]);
      }
    }
    // attn rows 0 and 1 past column 15 (Akk ran into them): positions
    // perm_pos(16…31) are the upper halves of the first four 8-position
    // groups, perm_pos(32…63) the last four groups.
    if (tid < 16) {
      const int zr = tid >> 3, g8 = tid & 7;
      if (g8 < 4)
        *reinterpret_cast<uint2*>(&T.At[tile_at<kL>(zr, 8 * g8 + 4)]) = make_uint2(0u, 0u);
      else
        *reinterpret_cast<uint4*>(&T.At[tile_at<kL>(zr, 8 * g8)]) = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  // Kcᵀ of chunk c (once T in fp32 has been read out of its slot): thread
  // (pair, a, mh) scales key channels dp, dp+1 of tokens 16m + 4a + e
  // (m = 2mh, 2mh+1; e = 0…3), one 32-bit read per token. Its tokens share
  // the row swizzle for each e (t mod 16 = 4a + e), so the reads differ by
  // immediate offsets, and each m gives four consecutive positions of
  // perm_pos: one 8-byte write per channel.
  auto finish_kc = [&](auto P) {
    constexpr int c = decltype(P)::value;
    const int tid = opaque(threadIdx.x);
    FusedTiles<K>& T = sh.buf[c];
    const int dp = 2 * (tid & 63), a4 = 4 * ((tid >> 6) & 3), mh = tid >> 8;
    const int rho0 = perm_inv(dp), rho1 = perm_inv(dp + 1);
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int t0 = 16 * (2 * mh + mm) + a4;
      const float4 s = *reinterpret_cast<const float4*>(&sh.gex[c][t0]);
      const float sc[4] = {s.x, s.y, s.z, s.w};
      float v0[4], v1[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(&T.Kt[tile_at<K>(t0 + e, dp)]);
        v0[e] = lo_f(w) * sc[e];
        v1[e] = hi_f(w) * sc[e];
      }
      const int pos = perm_pos(t0);
      *reinterpret_cast<uint2*>(&T.Kc[tile_at<kL>(rho0, pos)]) =
          make_uint2(pk_bf16(v0[0], v0[1]), pk_bf16(v0[2], v0[3]));
      *reinterpret_cast<uint2*>(&T.Kc[tile_at<kL>(rho1, pos)]) =
          make_uint2(pk_bf16(v1[0], v1[1]), pk_bf16(v1[2], v1[3]));
    }
  };

  // =========================================================================
  // Scan state and the scan's phases
  // =========================================================================
  const int jw = tile * kBW + 16 * wave;  // this wave's first value column
  const int jl = jw + r16;                // this lane's column (accumulator layout)

  // S[:, jw…jw+15] in accumulator layout: tile rb, row m holds key channel
  // perm_pos(16·rb + m).
  f32x4 S[RBK];
  {
    const float* sin = p.s_in + size_t(bh) * K * p.V + jl;
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[rb][r] = sin[size_t(perm_pos(16 * rb + 4 * q4 + r)) * p.V];
  }
  // v of this lane's 16 tokens, read as 32-bit words of two adjacent
  // columns: in each pair of lanes (columns c, c+1) the even lane reads
  // token t's word (v[t][c], v[t][c+1]) and the odd lane token t+1's; a swap
  // of halves between the two lanes (vpair) then gives each its column at
  // tokens t, t+1. Eight word loads stay in flight together, where sixteen
  // 16-bit loads packed in pairs would each wait for the one before.
  uint32_t vA[4][2];
  const int HV = p.H * p.V;
  const int vcol = jw + (r16 & ~1), vtok = 4 * q4 + (r16 & 1);
  // Byte offset of this lane's first word within a chunk's v rows.
  const uint32_t vlane = 2u * (uint32_t(vtok) * uint32_t(HV) + uint32_t(vcol));
  auto load_v = [&](int n) {
    const int rl = min(kL, p.S - n * kL);
    const uint16_t* vb = p.v + (bh_row0 + size_t(n) * kL * tokstride) * p.V;
    if (rl == kL) {
      // A whole chunk: raw buffer loads over its rows, the lane offset fixed
      // and the token's offset a scalar (no per-load address arithmetic).
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(vb), 0, 0x7fffffff, 0x00020000);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2)
          vA[tb][r2] = __builtin_amdgcn_raw_buffer_load_b32(
              rs, vlane, 2u * uint32_t(16 * tb + 2 * r2) * uint32_t(HV), 0);
    } else {
      // The last, partial chunk: tokens clamped to its last row (offsets
      // grow with the token, so that is clamping the offset).
      const uint32_t vlast = 2u * (uint32_t((rl - 1) * HV) + uint32_t(vcol));
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) {
          const uint32_t o =
              min(vlane + 2u * uint32_t(16 * tb + 2 * r2) * uint32_t(HV), vlast);
          vA[tb][r2] =
              *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(vb) + o);
        }
    }
  };
  // (v[t][c], v[t+1][c]) for this lane's column c from the lane pair's words.
  const uint32_t vsel = (r16 & 1) ? 0x03020706u : 0x05040100u;
  auto vpair = [&](uint32_t w) {
    const uint32_t other = uint32_t(__builtin_amdgcn_mov_dpp(int(w), 0xB1, 0xf, 0xf, false));
    return __builtin_amdgcn_perm(other, w, vsel);
  };
  auto as8 = [](const uint4& x) { return __builtin_bit_cast(bf16x8, x); };

  f32x4 X[4], yt[4], Vp[4];
  uint4 vf[2];
  // Phase 1 over k-steps kk0 … kk0+1: X += K·S and yᵀ += Sᵀ·Qᵀ from the same S
  // fragments (hi, lo); fragment reads run one step ahead of the MFMAs.
  auto phase1 = [&](const FusedTiles<K>& T, int kk0) {
    const int lane = opaque(tid) & 63, r16 = lane & 15, k8 = 8 * (lane >> 4);
    bf16x8 kf[2], qf[2];
    kf[0] = ld8(&T.Kt[tile_at<K>(r16, 32 * kk0 + k8)]);
    qf[0] = ld8(&T.Qt[tile_at<K>(r16, 32 * kk0 + k8)]);
#pragma unroll
    for (int kq = 0; kq < 2; ++kq) {
      const int kk = kk0 + kq;
      const uint4 shi = frag_hi(S[2 * kk], S[2 * kk + 1]);
      const uint4 slo = frag_lo(S[2 * kk], S[2 * kk + 1], shi);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int st = 4 * kq + tb, nx = st + 1;
        if (nx < 8) {
          const int at = tile_at<K>(16 * (nx & 3) + r16, 32 * (kk0 + (nx >> 2)) + k8);
          kf[nx & 1] = ld8(&T.Kt[at]);
          qf[nx & 1] = ld8(&T.Qt[at]);
        }
        X[tb] = mfma16(kf[st & 1], as8(shi), X[tb]);
        X[tb] = mfma16(kf[st & 1], as8(slo), X[tb]);
        yt[tb] = mfma16(as8(shi), qf[st & 1], yt[tb]);
      }
    }
  };

  // =========================================================================
  // Prologue: chunk 0 built by all waves; S and chunk 0's v loaded
  // =========================================================================
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // vmcnt(0): this wave's loads, its HBM → LDS copies included, have landed.
  auto wait_loads = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };
  // attn's blocks above the diagonal, in both buffers: zero for every chunk.
  for (int i = tid; i < 2 * kL * kL / 8; i += kT)
    *reinterpret_cast<uint4*>(&sh.buf[i / (kL * kL / 8)].At[8 * (i % (kL * kL / 8))]) =
        make_uint4(0u, 0u, 0u, 0u);
  dma_kq(P0{}, 0);
  load_gates(0);
  wait_loads();
  __syncthreads();
  put_gates(P0{});
  if (p.N > 1) {
    dma_kq(P1{}, 1);
    load_gates(1);
  }
  __syncthreads();
  scores(P0{});
  __syncthreads();
  diag(P0{});
  if (p.N > 1) {
    // chunk 1's gates (scores of chunk 0 have read the shared G and erase)
    wait_loads();
    put_gates(P1{});
  }
  __syncthreads();
  merge_step1(Abuf(P0{}), Tbuf(P0{}), sh.xw[0], wave, lane);
  __syncthreads();
  merge_steps23(Abuf(P0{}), Tbuf(P0{}), sh.xw[wave & 3], wave, lane);
  __syncthreads();
  finish_t(P0{});
  load_v(0);
  __syncthreads();

  // One chunk: the scan of chunk n from buffer CUR, the build of chunk n+1
  // into the other.
  auto chunk = [&](auto CURC, int n) {
    constexpr int cur = decltype(CURC)::value;
    using NX = std::integral_constant<int, 1 - cur>;
    const FusedTiles<K>& T = sh.buf[cur];
    const bool more = n + 1 < p.N;   // chunk n+1 is built in this iteration

    // --- a: Kcᵀ(n) ‖ k-steps 0-1
    finish_kc(CURC);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      X[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
      yt[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    phase1(T, 0);
    wait_loads();  // chunk n+1's K and Q have landed in LDS
    lds_barrier();

    // --- b: scores of chunk n+1 ‖ k-steps 2-3, X, v of chunk n+1
    if (more) scores(NX{});
    phase1(T, 2);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      float gw[4], ge[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        gw[r] = sh.gwr[cur][16 * tb + 4 * q4 + r];
        ge[r] = sh.gxe[cur][16 * tb + 4 * q4 + r];
      }
      const uint32_t vp[2] = {vpair(vA[tb][0]), vpair(vA[tb][1])};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float vv = (r & 1) ? hi_f(vp[r >> 1]) : lo_f(vp[r >> 1]);
        X[tb][r] = gw[r] * vv - ge[r] * X[tb][r];
      }
      const float ysc = sh.gys[cur][16 * tb + r16];
#pragma unroll
      for (int r = 0; r < 4; ++r) yt[tb][r] *= ysc;
    }
    load_v(more ? n + 1 : n);
    lds_barrier();

    // --- c: chunk n+2's K and Q into chunk n's (now read) slots, its gates;
    // diagonal inverses of chunk n+1 ‖ V' = T·X (hi + lo parts of both)
    if (n + 2 < p.N) {
      dma_kq(CURC, n + 2);
      load_gates(n + 2);
    }
    if (more) diag(NX{});
    {
      uint4 xh[2], xl[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        xh[kk] = frag_hi(X[2 * kk], X[2 * kk + 1]);
        xl[kk] = frag_lo(X[2 * kk], X[2 * kk + 1], xh[kk]);
      }
      // T is lower triangular: its six nonzero (row block, k-step) pairs.
      auto at = [&](int st) { return tile_at<kL>(16 * tril_tb(st) + r16, 32 * tril_kk(st) + k8); };
      bf16x8 th[2], tlo[2];
      th[0] = ld8(&T.Th[at(0)]);
      tlo[0] = ld8(&T.Tl[at(0)]);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) Vp[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kTriSteps; ++st) {
        if (st + 1 < kTriSteps) {
          th[(st + 1) & 1] = ld8(&T.Th[at(st + 1)]);
          tlo[(st + 1) & 1] = ld8(&T.Tl[at(st + 1)]);
        }
        const int tb = tril_tb(st), kk = tril_kk(st);
        Vp[tb] = mfma16(th[st & 1], as8(xh[kk]), Vp[tb]);
        Vp[tb] = mfma16(tlo[st & 1], as8(xh[kk]), Vp[tb]);
        Vp[tb] = mfma16(th[st & 1], as8(xl[kk]), Vp[tb]);
      }
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) vf[kk] = frag_hi(Vp[2 * kk], Vp[2 * kk + 1]);
    }
    lds_barrier();

    // --- d: merge step 1 of chunk n+1 (waves 0, 1) ‖ S decay,
    // yᵀ += V'ᵀ·attnᵀ, S += Kcᵀ·V' for state rows 0-63
    if (more) merge_step1(Abuf(NX{}), Tbuf(NX{}), sh.xw[0], wave, opaque(lane));
    {
      const float egl = sh.gegl[cur][0];
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[rb][r] *= egl;
      // attn is lower triangular too.
      auto at = [&](int st) { return tile_at<kL>(16 * tril_tb(st) + r16, 32 * tril_kk(st) + k8); };
      bf16x8 fr[2];
      fr[0] = ld8(&T.At[at(0)]);
#pragma unroll
      for (int st = 0; st < kTriSteps; ++st) {
        if (st + 1 < kTriSteps) fr[(st + 1) & 1] = ld8(&T.At[at(st + 1)]);
        yt[tril_tb(st)] = mfma16(as8(vf[tril_kk(st)]), fr[st & 1], yt[tril_tb(st)]);
      }
    }
    // S += Kcᵀ·V' for state row blocks rb0 … rb0+3
    auto state_update = [&](int rb0) {
      bf16x8 fr[2];
      fr[0] = ld8(&T.Kc[tile_at<kL>(16 * rb0 + r16, k8)]);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (st + 1 < 8)
          fr[(st + 1) & 1] = ld8(
              &T.Kc[tile_at<kL>(16 * (rb0 + ((st + 1) >> 1)) + r16, 32 * ((st + 1) & 1) + k8)]);
        S[rb0 + (st >> 1)] = mfma16(fr[st & 1], as8(vf[st & 1]), S[rb0 + (st >> 1)]);
      }
    };
    state_update(0);
    lds_barrier();

    // --- e: merge steps 2 and 3 of chunk n+1 (waves 0-3) ‖ S += Kcᵀ·V' for
    // rows 64-127, y
    if (more) merge_steps23(Abuf(NX{}), Tbuf(NX{}), sh.xw[wave & 3], wave, opaque(lane));
    state_update(4);
    {
      // y: lane (r16, q4) holds columns jw + 4q4 … +3 of token 16tb + r16;
      // rows past the sequence end go to the sink row.
      TY* yb = static_cast<TY*>(p.y) + (bh_row0 + size_t(n) * kL * tokstride) * p.V;
      const int rl = p.S - n * kL;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int t = 16 * tb + r16;
        TY* dst = t < rl ? reinterpret_cast<TY*>(reinterpret_cast<char*>(yb) +
                                                 sizeof(TY) * uint32_t(t * HV + jw + 4 * q4))
                         : reinterpret_cast<TY*>(p.sink) + jw + 4 * q4;
        if constexpr (sizeof(TY) == 2)
          *reinterpret_cast<uint2*>(dst) =
              make_uint2(pk_bf16(yt[tb][0], yt[tb][1]), pk_bf16(yt[tb][2], yt[tb][3]));
        else
          *reinterpret_cast<float4*>(dst) =
              make_float4(yt[tb][0], yt[tb][1], yt[tb][2], yt[tb][3]);
      }
    }
    lds_barrier();

    // --- f: T hi/lo and attn of chunk n+1; the gates of chunk n+2 into this
    // chunk's gate buffer (its last reader was segment d). Chunk n+1's Kcᵀ
    // follows in the next chunk's segment a, once every wave has read T out
    // of its slot.
    if (more) finish_t(NX{});
    if (n + 2 < p.N) put_gates(CURC);
    lds_barrier();
  };

  for (int n = 0; n < p.N; n += 2) {
    chunk(P0{}, n);
    if (n + 1 < p.N) chunk(P1{}, n + 1);
  }

  float* sout = p.s_out + size_t(bh) * K * p.V + jl;
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) sout[size_t(perm_pos(16 * rb + 4 * q4 + r)) * p.V] = S[rb][r];
}

size_t region(size_t bytes) { return align_up(bytes, 256); }

}  // namespace

// The fused kernel covers per-head gates (erase and write of width 1, decay
// of width 0 or 1) at head_k_dim 128, head_v_dim a multiple of 128, chunk 64,
// bf16 q/k/v.
bool fused_fwd_supported(const Dims& d, int qkv_dtype) {
  return qkv_dtype == DN_BF16 && d.K == 128 && d.V % kBW == 0 && d.L == kL && d.ew == 1 &&
         d.ww == 1 && d.dw <= 1 && token_rows_fit_32bit(d);
}

// The sink row: the target of y rows past the sequence end.
size_t fused_fwd_workspace(const Dims& d) { return region(size_t(d.V) * 4); }

hipError_t fused_fwd(const Dims& d, int y_dtype, const void* q, const void* k, const void* v,
                     const float* erase, const float* write, const float* g,
                     const float* state_in, void* y, float* state_out, void* ws,
                     hipStream_t stream) {
  FusedParams p;
  p.B = d.B;
  p.S = d.S;
  p.H = d.H;
  p.V = d.V;
  p.N = d.N;
  p.scale = d.scale;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.erase = erase;
  p.write = write;
  p.g = g;
  p.s_in = state_in;
  p.y = y;
  p.s_out = state_out;
  p.sink = static_cast<uint16_t*>(ws);
  const unsigned blocks = unsigned(((d.B * d.H + 7) / 8) * 8 * (d.V / kBW));
  ProfScope ps("dn_mfma_fused", stream);
#define DN_FUSED(TY, GT)                                                                 \
  hipLaunchKernelGGL((fused_fwd_kernel<128, TY, GT>), dim3(blocks), dim3(kT), 0, stream, \
                     p)
  const bool gated = d.dw > 0;
  if (y_dtype == DN_BF16) {
    if (gated) DN_FUSED(bf16, true); else DN_FUSED(bf16, false);
  } else {
    if (gated) DN_FUSED(float, true); else DN_FUSED(float, false);
  }
#undef DN_FUSED
  return hipGetLastError();
}

}  // namespace dn
