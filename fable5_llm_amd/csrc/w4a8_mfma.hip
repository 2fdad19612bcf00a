// Batched W4A8 (several tokens): int8 MFMA on gfx950 with the per-group
// scale applied after accumulation.  Per token the result is bit-identical
// to ref/w4a8_ref.py:254-289 matvec_y32: every group sum is exact in int32
// (|16 * sum w*x| <= 2^21) and the scale products are summed in int64.
//
// v_mfma_i32_16x16x64_i8: A = 16 weight rows x 64 k, B = 64 k x 16 tokens,
// D = 16 x 16 int32.  Lane l feeds row/token (l % 16) and k-quarter l / 16
// of A and B alike, so A and B share one lane->k mapping and the dot product
// does not depend on the order in which the hardware walks k.  D element
// (4 * (l / 16) + r, l % 16) lands in lane l, register r.
#include "w4a8_internal.h"

namespace w4a8 {

typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int kMaxColTiles = 4;   // B <= 64

__device__ __forceinline__ int cvt_lo16(uint32_t w) {
  // offset-form low nibbles u = w + 8 -> bytes 16*w (exact int8)
  return (int)(((w << 4) & 0xF0F0F0F0u) ^ 0x80808080u);
}
__device__ __forceinline__ int cvt_hi16(uint32_t w) {
  return (int)(w & 0xF0F0F0F0u);   // two's-complement high nibbles -> 16*w
}

__device__ __forceinline__ int64_t rshr64_mm(int64_t v, int s) {
  if (s == 0) return v;
  const int64_t half = (int64_t)1 << (s - 1);
  return v >= 0 ? ((v + half) >> s) : -((-v + half) >> s);
}

__global__ __launch_bounds__(kWG) void matmul_kernel(
    const uint8_t *W, int32_t nrows, int64_t ntiles, int64_t tile_bytes, int NG,
    int nblk, int sh, const int8_t *x8, int B, int K, int32_t *y32,
    int32_t *err) {
  __shared__ int64_t red[kWaves - 1][kMaxColTiles][4][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, c = lane & 15;
  const int CT = (B + 15) / 16;
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    const uint8_t *tb = W + t * tile_bytes;
    int64_t p[kMaxColTiles][4];
#pragma unroll
    for (int ct = 0; ct < kMaxColTiles; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) p[ct][r] = 0;
    for (int b = wave; b < nblk; b += kWaves) {
      const uint8_t *bb = tb + (int64_t)b * kBlockBytes;
      uint4 sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = ldg16_nt(bb + (4 * q + r) * 16);
      const int ng = min(kGroupsPerBlock, NG - b * kGroupsPerBlock);
      for (int i = 0; i < ng; ++i) {
        const int g = b * kGroupsPerBlock + i;
        const uint4 wp = ldg16_nt(bb + kScaleChunk + i * kGroupChunk + (c * 4 + q) * 16);
        const v4i a0 = {cvt_lo16(wp.x), cvt_hi16(wp.x), cvt_lo16(wp.y), cvt_hi16(wp.y)};
        const v4i a1 = {cvt_lo16(wp.z), cvt_hi16(wp.z), cvt_lo16(wp.w), cvt_hi16(wp.w)};
        uint32_t m[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t w = (i >> 1) == 0 ? sc[r].x
                           : (i >> 1) == 1 ? sc[r].y
                           : (i >> 1) == 2 ? sc[r].z : sc[r].w;
          m[r] = (i & 1) ? (w >> 16) : (w & 0xFFFFu);
        }
#pragma unroll
        for (int ct = 0; ct < kMaxColTiles; ++ct) {
          if (ct < CT) {
            const int tok = ct * 16 + c;
            v4i b0 = {0, 0, 0, 0}, b1 = {0, 0, 0, 0};
            if (tok < B) {
              const int8_t *xp = x8 + (int64_t)tok * K + kGroup * g + 32 * q;
              const int4 u0 = *(const int4 *)xp, u1 = *(const int4 *)(xp + 16);
              b0 = v4i{u0.x, u0.y, u0.z, u0.w};
              b1 = v4i{u1.x, u1.y, u1.z, u1.w};
            }
            v4i acc = {0, 0, 0, 0};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              p[ct][r] += (int64_t)(int32_t)m[r] * (int64_t)acc[r];
          }
        }
      }
    }
    if (wave > 0) {
#pragma unroll
      for (int ct = 0; ct < kMaxColTiles; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave - 1][ct][r][lane] = p[ct][r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int ct = 0; ct < kMaxColTiles; ++ct) {
        if (ct < CT) {
          const int tok = ct * 16 + c;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int64_t tot = p[ct][r];
#pragma unroll
            for (int w = 0; w < kWaves - 1; ++w) tot += red[w][ct][r][lane];
            const int64_t row = t * kTileRows + 4 * q + r;
            if (tok < B && row < nrows) {
              const int64_t y = rshr64_mm(tot >> 4, sh);
              if (y > 2147483647LL || y < -2147483647LL) atomicOr(err, 1);
              y32[(int64_t)tok * nrows + row] = (int32_t)y;
            }
          }
        }
      }
    }
    __syncthreads();
  }
}

hipError_t launch_matmul(const uint8_t *w, int32_t nrows, const Layout &L, int32_t sh,
                         const int8_t *x8, int32_t B, int32_t *y32, int32_t *err,
                         hipStream_t s) {
  const int64_t ntiles = (nrows + kTileRows - 1) / kTileRows;
  int dev = 0, ncu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t cap = (int64_t)ncu * 4;
  const int grid = (int)(ntiles < cap ? ntiles : cap);
  hipLaunchKernelGGL(matmul_kernel, dim3(grid), dim3(kWG), 0, s, w, nrows, ntiles,
                     L.tile_bytes, L.NG, L.nblk, sh, x8, B, L.K, y32, err);
  return hipGetLastError();
}

}  // namespace w4a8
