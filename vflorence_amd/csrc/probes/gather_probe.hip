// Read-only probe of the cross-attention access pattern (measurement only: bench.py
// --gather-probe; nothing in the ops calls it).  Every group's pages, all 16 heads, K
// and V, are XOR-folded into one value per workgroup, stored only if it hits a sentinel.
// The variants differ only in which workgroup and wave read which slices of a block.
#include <hip/hip_runtime.h>
#include <stdint.h>

// pages: [G][W] int32; nb: [G] blocks per group; pools k, v: [NB][16 heads][16 tok][64] bf16
// slice (block, head) = 2 KiB at ((page * 16 + h) * 1024) elements.
struct Args {
  const uint16_t *k, *v;
  const int32_t *pages, *nb, *order;
  int W, G;
  uint32_t *out;
};

__device__ __forceinline__ uint32_t fold(uint4 a) { return a.x ^ a.y ^ a.z ^ a.w; }

// A: workgroup = (group, head); 4 waves split the group's blocks into contiguous runs;
// each wave loads 2 blocks (K and V, 2 KiB each) per iteration.
// MAP 0: id -> (id / 16, id % 16)  (current kernel)   MAP 1: id -> (id % G, id / G)
template <int MAP>
__global__ __launch_bounds__(256) void probe_slices(Args a) {
  int id = blockIdx.x;
  int g, h;
  if (MAP == 0) { g = id / 16; h = id % 16; } else { g = id % a.G; h = id / a.G; }
  g = a.order[g];
  const int n = a.nb[g];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lo = n * wave / 4, hi = n * (wave + 1) / 4;
  uint32_t acc = 0;
  const int32_t *pg = a.pages + (int64_t)g * a.W;
  for (int i = lo; i < hi; i += 2) {
    uint4 r[8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = i + u < hi ? pg[i + u] : pg[i];
      const int64_t base = ((int64_t)b * 16 + h) * 1024 + lane * 8;
      const uint4 *kp = (const uint4 *)(a.k + base), *vp = (const uint4 *)(a.v + base);
      r[u * 4 + 0] = kp[0]; r[u * 4 + 1] = kp[64];
      r[u * 4 + 2] = vp[0]; r[u * 4 + 3] = vp[64];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= fold(r[j]);
  }
  if (acc == 0x12345678u) a.out[id] = acc;
}

// A with non-temporal loads (the hint the attention kernels use for K/V pages).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt(const uint4 *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__global__ __launch_bounds__(256) void probe_slices_nt(Args a) {
  int id = blockIdx.x;
  int g = a.order[id / 16], h = id % 16;
  const int n = a.nb[g];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lo = n * wave / 4, hi = n * (wave + 1) / 4;
  uint32_t acc = 0;
  const int32_t *pg = a.pages + (int64_t)g * a.W;
  for (int i = lo; i < hi; i += 2) {
    uint4 r[8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = i + u < hi ? pg[i + u] : pg[i];
      const int64_t base = ((int64_t)b * 16 + h) * 1024 + lane * 8;
      const uint4 *kp = (const uint4 *)(a.k + base), *vp = (const uint4 *)(a.v + base);
      r[u * 4 + 0] = ld_nt(kp); r[u * 4 + 1] = ld_nt(kp + 64);
      r[u * 4 + 2] = ld_nt(vp); r[u * 4 + 3] = ld_nt(vp + 64);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= fold(r[j]);
  }
  if (acc == 0x12345678u) a.out[id] = acc;
}

// A with non-temporal loads, NW waves per workgroup and UB blocks per iteration (the
// cross-attention kernel runs eight waves and two blocks per stage).
template <int NW, int UB>
__global__ __launch_bounds__(NW * 64) void probe_slices_ntw(Args a) {
  int id = blockIdx.x;
  int g = a.order[id / 16], h = id % 16;
  const int n = a.nb[g];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lo = n * wave / NW, hi = n * (wave + 1) / NW;
  uint32_t acc = 0;
  const int32_t *pg = a.pages + (int64_t)g * a.W;
  for (int i = lo; i < hi; i += UB) {
    uint4 r[4 * UB];
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int b = i + u < hi ? pg[i + u] : pg[i];
      const int64_t base = ((int64_t)b * 16 + h) * 1024 + lane * 8;
      const uint4 *kp = (const uint4 *)(a.k + base), *vp = (const uint4 *)(a.v + base);
      r[u * 4 + 0] = ld_nt(kp); r[u * 4 + 1] = ld_nt(kp + 64);
      r[u * 4 + 2] = ld_nt(vp); r[u * 4 + 3] = ld_nt(vp + 64);
    }
#pragma unroll
    for (int j = 0; j < 4 * UB; ++j) acc ^= fold(r[j]);
  }
  if (acc == 0x12345678u) a.out[id] = acc;
}

// A with non-temporal loads and the 16 heads of each group on one XCD: workgroup ids go
// to the 8 XCDs round robin (id % 8), so XCD x takes the order positions x, x + 8, ...,
// each for all 16 heads (a block's 32 KiB of K, and of V, read through one L2).
__global__ __launch_bounds__(256) void probe_slices_xcd(Args a) {
  const int id = blockIdx.x;
  const int x = id % 8, j = id / 8;
  const int pos = 8 * (j / 16) + x;
  if (pos >= a.G) return;
  const int g = a.order[pos], h = j % 16;
  const int n = a.nb[g];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lo = n * wave / 4, hi = n * (wave + 1) / 4;
  uint32_t acc = 0;
  const int32_t *pg = a.pages + (int64_t)g * a.W;
  for (int i = lo; i < hi; i += 2) {
    uint4 r[8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = i + u < hi ? pg[i + u] : pg[i];
      const int64_t base = ((int64_t)b * 16 + h) * 1024 + lane * 8;
      const uint4 *kp = (const uint4 *)(a.k + base), *vp = (const uint4 *)(a.v + base);
      r[u * 4 + 0] = ld_nt(kp); r[u * 4 + 1] = ld_nt(kp + 64);
      r[u * 4 + 2] = ld_nt(vp); r[u * 4 + 3] = ld_nt(vp + 64);
    }
#pragma unroll
    for (int j2 = 0; j2 < 8; ++j2) acc ^= fold(r[j2]);
  }
  if (acc == 0x12345678u) a.out[pos * 16 + h] = acc;
}

// B: workgroup = (group, quad of 4 heads), 16 waves: wave = (head in quad, run).
__global__ __launch_bounds__(1024) void probe_quads(Args a) {
  int id = blockIdx.x;
  int g = a.order[id / 4], q = id % 4;
  const int n = a.nb[g];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int h = q * 4 + wave / 4, run = wave % 4;
  const int lo = n * run / 4, hi = n * (run + 1) / 4;
  uint32_t acc = 0;
  const int32_t *pg = a.pages + (int64_t)g * a.W;
  for (int i = lo; i < hi; i += 2) {
    uint4 r[8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = i + u < hi ? pg[i + u] : pg[i];
      const int64_t base = ((int64_t)b * 16 + h) * 1024 + lane * 8;
      const uint4 *kp = (const uint4 *)(a.k + base), *vp = (const uint4 *)(a.v + base);
      r[u * 4 + 0] = kp[0]; r[u * 4 + 1] = kp[64];
      r[u * 4 + 2] = vp[0]; r[u * 4 + 3] = vp[64];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= fold(r[j]);
  }
  if (acc == 0x12345678u) a.out[id] = acc;
}

// C: workgroup = (group, quad), 4 waves; wave = run; each wave reads the 4 heads' slices
// of its blocks: 8 KiB contiguous per block per tensor (8 loads of 1 KiB).
__global__ __launch_bounds__(256) void probe_quads_wave(Args a) {
  int id = blockIdx.x;
  int g = a.order[id / 4], q = id % 4;
  const int n = a.nb[g];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lo = n * wave / 4, hi = n * (wave + 1) / 4;
  uint32_t acc = 0;
  const int32_t *pg = a.pages + (int64_t)g * a.W;
  for (int i = lo; i < hi; ++i) {
    const int b = pg[i];
    const int64_t base = ((int64_t)b * 16 + q * 4) * 1024 + lane * 8;
    const uint4 *kp = (const uint4 *)(a.k + base), *vp = (const uint4 *)(a.v + base);
    uint4 r[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) { r[j] = kp[j * 64]; r[8 + j] = vp[j * 64]; }
#pragma unroll
    for (int j = 0; j < 16; ++j) acc ^= fold(r[j]);
  }
  if (acc == 0x12345678u) a.out[id] = acc;
}

extern "C" int probe_launch(int variant, const void *k, const void *v, const int32_t *pages,
                            const int32_t *nb, const int32_t *order, int W, int G,
                            uint32_t *out, void *stream) {
  Args a{(const uint16_t *)k, (const uint16_t *)v, pages, nb, order, W, G, out};
  hipStream_t s = (hipStream_t)stream;
  switch (variant) {
    case 0: probe_slices<0><<<G * 16, 256, 0, s>>>(a); break;
    case 1: probe_slices<1><<<G * 16, 256, 0, s>>>(a); break;
    case 2: probe_quads<<<G * 4, 1024, 0, s>>>(a); break;
    case 3: probe_quads_wave<<<G * 4, 256, 0, s>>>(a); break;
    case 4: probe_slices_nt<<<G * 16, 256, 0, s>>>(a); break;
    case 5: probe_slices_ntw<8, 2><<<G * 16, 512, 0, s>>>(a); break;
    case 6: probe_slices_ntw<8, 4><<<G * 16, 512, 0, s>>>(a); break;
    case 7: probe_slices_ntw<16, 2><<<G * 16, 1024, 0, s>>>(a); break;
    case 8: probe_slices_xcd<<<(G + 7) / 8 * 8 * 16, 256, 0, s>>>(a); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
