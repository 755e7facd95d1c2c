// Attention kernels for the reference's head sizes other than 64 and 128
// (vflorence/layers/attention.py:6: 32, 48, 80, 96, 112, 160, 192, 224, 256, 512), in a
// translation unit of their own so they compile in parallel with the rest.
//
// What runs: fp32 caches on the VALU kernel (decode_valu.h, lanes padded to a power of
// two per token row); 16-bit caches on the one-row / shared-table matrix-core kernel
// (decode_mfma.h, the last 32-wide K chunk masked when the head size is not a multiple
// of 32).  Wave counts are fixed per head size -- four up to 128, two up to 256, one for
// 512 -- so the cross-wave merge buffer stays within 64 KiB of LDS and a wave's
// registers (a 512-wide head holds 320 VGPRs of K/V, query and sums) fit; one block per
// stage above 128.  A call asking for one wave gets one wave.
#include "attention_dispatch.h"

namespace vfl {

template <int D> constexpr int other_waves() { return D <= 128 ? 4 : (D <= 256 ? 2 : 1); }
template <int D> constexpr int other_stage_blocks() { return D <= 128 ? 2 : 1; }

template <int D>
static int valu_other(const AttnArgs &a, int gmax, int nw) {
  constexpr int NW = other_waves<D>();
  if (nw <= 1 || NW == 1) {
    if (gmax <= 1) return launch_valu<D, 1, 1>(a);
    if (gmax <= 2) return launch_valu<D, 2, 1>(a);
    if (gmax <= 4) return launch_valu<D, 4, 1>(a);
    return launch_valu<D, 8, 1>(a);
  }
  if (gmax <= 1) return launch_valu<D, 1, NW>(a);
  if (gmax <= 2) return launch_valu<D, 2, NW>(a);
  if (gmax <= 4) return launch_valu<D, 4, NW>(a);
  return launch_valu<D, 8, NW>(a);
}

template <int DT, int D>
static int mfma_other(const AttnArgs &a, int nw) {
  constexpr int NW = other_waves<D>(), U = other_stage_blocks<D>();
  if (nw <= 1 || NW == 1) return launch_mfma_rows<DT, D, 1, U>(a);
  return launch_mfma_rows<DT, D, NW, U>(a);
}

template <int D>
static int other_dim(const AttnArgs &a, int dtype, int gmax, int nw) {
  if (dtype == VFL_FLOAT32) return valu_other<D>(a, gmax, nw);
  if (dtype == VFL_BFLOAT16) return mfma_other<VFL_BFLOAT16, D>(a, nw);
  return mfma_other<VFL_FLOAT16, D>(a, nw);
}

int dispatch_other_head_dim(const AttnArgs &a, int dtype, int head_dim, int gmax, int nw) {
  switch (head_dim) {
    case 32: return other_dim<32>(a, dtype, gmax, nw);
    case 48: return other_dim<48>(a, dtype, gmax, nw);
    case 80: return other_dim<80>(a, dtype, gmax, nw);
    case 96: return other_dim<96>(a, dtype, gmax, nw);
    case 112: return other_dim<112>(a, dtype, gmax, nw);
    case 160: return other_dim<160>(a, dtype, gmax, nw);
    case 192: return other_dim<192>(a, dtype, gmax, nw);
    case 224: return other_dim<224>(a, dtype, gmax, nw);
    case 256: return other_dim<256>(a, dtype, gmax, nw);
    case 512: return other_dim<512>(a, dtype, gmax, nw);
    default:
      set_error("attention_with_kv_cache: head_dim %d has no kernel", head_dim);
      return VFL_E_UNSUPPORTED;
  }
}

}  // namespace vfl
