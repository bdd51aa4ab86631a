// The chunk scan with OutNorm (norm.rs:106-144) in its y write: the NORM
// instantiations of mfma_scan_kernel (mfma_scan.hpp), compiled apart from
// the plain scan so the two translation units build in parallel. The
// launches are in chunk_fwd_mfma.hip (mfma_fwd_norm).

#include "mfma_scan.hpp"

namespace dn {

const void* norm_scan_fn(int K, bool pc, bool seg, bool y_bf16, int waves, bool gated) {
#define DN_NK(KD, TY, W, PCV, SG)                                                                 \
  do {                                                                                            \
    if (gated)                                                                                    \
      return reinterpret_cast<const void*>(&mfma_scan_kernel<KD, TY, W, PCV, false, SG, 2>);      \
    return reinterpret_cast<const void*>(&mfma_scan_kernel<KD, TY, W, PCV, false, SG, 1>);        \
  } while (0)
#define DN_NK_W(KD, TY, PCV, SG)               \
  do {                                         \
    if (waves == 8) DN_NK(KD, TY, 8, PCV, SG); \
    if (waves == 4) DN_NK(KD, TY, 4, PCV, SG); \
    DN_NK(KD, TY, 2, PCV, SG);                 \
  } while (0)
#define DN_NK_PC(KD, TY, SG)           \
  do {                                 \
    if (pc) DN_NK_W(KD, TY, true, SG); \
    DN_NK_W(KD, TY, false, SG);        \
  } while (0)
  if (seg) {  // the segmented scan's output pass: 8 waves, head_k_dim 128
    if (y_bf16) {
      if (pc) DN_NK(128, bf16, 8, true, 2);
      DN_NK(128, bf16, 8, false, 2);
    }
    if (pc) DN_NK(128, float, 8, true, 2);
    DN_NK(128, float, 8, false, 2);
  }
  if (K == 128) {
    if (y_bf16) DN_NK_PC(128, bf16, 0);
    DN_NK_PC(128, float, 0);
  }
  if (y_bf16) DN_NK_PC(64, bf16, 0);
  DN_NK_PC(64, float, 0);
#undef DN_NK_PC
#undef DN_NK_W
#undef DN_NK
}

}  // namespace dn
