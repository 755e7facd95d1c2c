// Attention over pools of 32-token blocks, the reference's block size on x86
// (vflorence/config.py:42), for every head size the reference accepts
// (vflorence/layers/attention.py:6), in a translation unit of its own.
//
// The one-row / shared-table matrix-core kernel (bf16, fp16) and the VALU kernel (fp32)
// walk 16-token parts, two per block: part p of table entry e is chunk 2 e + p, at
// 16 * head_dim elements into the block-head slice in K and in the 4-token-interleaved
// V alike.  Own-table beam groups, group plans and the fused KV write are built for
// 16-token blocks; for these pools the entry points run every row as its own group and
// the write as its own launch.  Wave counts: one, or the size's fixed count (eight for
// 64, as the decode-step measurements chose for 16-token blocks; four for the other
// sizes up to 128, whose eight-wave merge buffer would pass 64 KiB of LDS at 128; two up
// to 256; one for 512); fp32 groups always take the eight-row kernel (a smaller group
// just leaves rows unused).
#include "attention_dispatch.h"

namespace vfl {

template <int D> constexpr int block32_waves() {
  return D == 64 ? 8 : (D <= 128 ? 4 : (D <= 256 ? 2 : 1));
}
template <int D> constexpr int block32_stage_blocks() { return D <= 128 ? 2 : 1; }

template <int D>
static int block32_dim(const AttnArgs &a, int dtype, int nw) {
  constexpr int NW = block32_waves<D>(), U = block32_stage_blocks<D>();
  const bool one = nw <= 1 || NW == 1;
  if (dtype == VFL_FLOAT32)
    return one ? launch_valu<D, 8, 1, 1>(a) : launch_valu<D, 8, (NW > 4 ? 4 : NW), 1>(a);
  if (dtype == VFL_BFLOAT16)
    return one ? launch_mfma_rows<VFL_BFLOAT16, D, 1, U, 1>(a)
               : launch_mfma_rows<VFL_BFLOAT16, D, NW, U, 1>(a);
  return one ? launch_mfma_rows<VFL_FLOAT16, D, 1, U, 1>(a)
             : launch_mfma_rows<VFL_FLOAT16, D, NW, U, 1>(a);
}

int dispatch_block32(const AttnArgs &a, int dtype, int head_dim, int gmax, int nw) {
  (void)gmax;  // every kernel here takes groups of up to 8 rows (16 on the matrix cores)
  switch (head_dim) {
    case 32: return block32_dim<32>(a, dtype, nw);
    case 48: return block32_dim<48>(a, dtype, nw);
    case 64: return block32_dim<64>(a, dtype, nw);
    case 80: return block32_dim<80>(a, dtype, nw);
    case 96: return block32_dim<96>(a, dtype, nw);
    case 112: return block32_dim<112>(a, dtype, nw);
    case 128: return block32_dim<128>(a, dtype, nw);
    case 160: return block32_dim<160>(a, dtype, nw);
    case 192: return block32_dim<192>(a, dtype, nw);
    case 224: return block32_dim<224>(a, dtype, nw);
    case 256: return block32_dim<256>(a, dtype, nw);
    case 512: return block32_dim<512>(a, dtype, nw);
    default:
      set_error("attention_with_kv_cache: head_dim %d has no kernel", head_dim);
      return VFL_E_UNSUPPORTED;
  }
}

}  // namespace vfl
