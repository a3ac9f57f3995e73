// Instantiations of the prefill attention kernel (fk_prefill_kernel.h) at the
// head sizes besides D = DV in {64, 128, 256}, bf16 pages and dense keys, kept
// in their own translation unit so that the two compile in parallel:
//   32      small encoders (L2/encoder_attention.py, hidden / heads = 384 / 12)
//   72      Qwen3-VL's vision encoder (1152 / 16; L2/vision_attention.py:32,39)
//   80      Qwen2-VL / Qwen2.5-VL's vision encoder (1280 / 16)
//   96      hidden / heads = 3072 / 32 models
//   192/128 MLA prefill: query / key 128 nope + 64 rope, value 128
//           (L2/mla_attention_impl.py:347-398 through FlashAttnVarlen)
#include "fk_prefill_kernel.h"

namespace fk {

bool launch_prefill_extra(int D, int DV, bool paged, bool split, const PrefillParams& P,
                          dim3 grid, const int32_t* bt, const int32_t* cu_q,
                          const int32_t* cu_k, hipStream_t stream) {
  if (D == DV) {
    switch (D) {
      case 32: launch_prefill_bf16<32, 32>(paged, split, P, grid, bt, cu_q, cu_k, stream); return true;
      case 72: launch_prefill_bf16<72, 72>(paged, split, P, grid, bt, cu_q, cu_k, stream); return true;
      case 80: launch_prefill_bf16<80, 80>(paged, split, P, grid, bt, cu_q, cu_k, stream); return true;
      case 96: launch_prefill_bf16<96, 96>(paged, split, P, grid, bt, cu_q, cu_k, stream); return true;
      default: return false;
    }
  }
  if (D == 192 && DV == 128) {
    launch_prefill_bf16<192, 128>(paged, split, P, grid, bt, cu_q, cu_k, stream);
    return true;
  }
  return false;
}

}  // namespace fk
