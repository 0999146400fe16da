// Bidirectional masked multi-head attention with the reference's softmax semantics, on MFMA.
//
// Reference: internal/embed/bert.go:356-402 with DotF32 / SoftmaxInPlace / fastExp
// (internal/ggml/ops_simd.go:46-97):
//   s = (q . k) * 1/sqrt(64);  mask[key] == 0  ->  s = -1e9 (assigned);
//   m = max s;  e = (s - m < -10) ? 0 : exp(s - m);  p = e / sum e;  o = sum p v.
// One block = 128 queries (64 when L <= 64) of one (sequence, head); one wave per 16 queries.
// Keys stream through LDS 64 at a time; S = K Q^T and O^T = V^T P^T run on
// v_mfma_f32_16x16x32_f16.
//
// Cutoff with an online max: a key is kept when s - m_run >= -10, with m_run the running max
// (tested exactly as a threshold on the unscaled score, keep_threshold). The exponentials use a
// reference point that trails m_run by a bounded amount, so the accumulators are rescaled only
// when the maximum moves far. Every key the reference keeps is kept (m_run <= m_final). A kept
// key the reference would drop has s - m_final < -10; the smallest kept score per query detects
// that case after the pass, and the block then repeats the pass with m_final fixed, which is
// exactly the reference rule.
// Key tiles outside [first valid key, last valid key] hold only masked keys; they contribute
// exact zeros and are skipped (all tiles are visited when a sequence has no valid key, where
// the reference's softmax is uniform).
//
// S-tile row permutation: S tile t row 4g+r holds key 32*(t/2) + 8g + 4*(t%2) + r, so the
// lane that owns rows 4g..4g+3 of tiles 2j and 2j+1 owns keys 32j + 8g .. 32j + 8g + 7 —
// exactly the 8 consecutive keys its B operand of the P.V MFMA needs. No cross-lane traffic.
#include "attention_device.h"

namespace lle {

template <int NW, bool EARLY>
__global__ __launch_bounds__(NW * 64, NW == 8 ? 4 : 1) void attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[AttnShape<NW>::LDS];
  // workgroup ids by the compiler builtins (see attention_dev's thread id)
  attention_dev<NW, EARLY>(a, __builtin_amdgcn_workgroup_id_x(), __builtin_amdgcn_workgroup_id_y(),
                           __builtin_amdgcn_workgroup_id_z(), lds);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
  // 128-query blocks read each key tile once per 128 queries; short sequences keep 64
  if (a.L > 64) {
    const dim3 grid((a.L + 127) / 128, a.H, a.B);
    if (a.L <= 512)
      hipLaunchKernelGGL((attention_kernel<8, true>), grid, dim3(512), 0, st, a);
    else
      hipLaunchKernelGGL((attention_kernel<8, false>), grid, dim3(512), 0, st, a);
  } else {
    const dim3 grid(1, a.H, a.B);
    hipLaunchKernelGGL((attention_kernel<4, true>), grid, dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace lle
