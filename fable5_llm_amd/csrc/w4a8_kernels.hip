// HIP kernels of the W4A8 matvec engine for gfx950 (MI355X).
//
// The integer law is the reference's: ref/w4a8_ref.py:254-289 (matvec_y32),
// ref/fixedpoint.py:24-75 (DYNQ8, rsqrt), ref/layer_fixed.py:1242-1278
// (RMSNorm), seq_model.py:1027-1050 + seq_movers.sv:759-836 (MOVY),
// gen_layer_script.py:1397-1433 (ALU ops, AMAX32).  Every product and sum is
// an exact integer, so any summation order gives bit-identical results.
#include <hip/hip_ext.h>

#include "w4a8_internal.h"

namespace w4a8 {

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t rshr64(int64_t v, int s) {
  // round half away from zero; s < 0 is an exact (wrapping) left shift.
  // Callers keep s within [-63, 63].
  if (s == 0) return v;
  if (s < 0) return (int64_t)((uint64_t)v << (-s));
  const int64_t half = (int64_t)1 << (s - 1);
  return v >= 0 ? ((v + half) >> s) : -((-v + half) >> s);
}

// MOVY dequant shift with the RTL caps: right by <= 63, left by <= 40
// (seq_movers.sv:770-777).
__device__ __forceinline__ int64_t movy_shift(int64_t v, int s) {
  if (s >= 0) return rshr64(v, s > 63 ? 63 : s);
  const int m = -s > 40 ? 40 : -s;
  return (int64_t)((uint64_t)v << m);
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// PWL sigmoid, Q12 in, Q15 out (fixedpoint.py:135-147).
__device__ __forceinline__ int32_t sigmoid_q(int32_t x, const int32_t *tab) {
  x = x < -(16 << 12) ? -(16 << 12) : (x > (16 << 12) - 1 ? (16 << 12) - 1 : x);
  const int32_t u = x + (16 << 12);
  const int32_t i = u >> 9, lo = u & 0x1FF;
  const int32_t a = tab[i], b = tab[i + 1];
  return a + (((b - a) * lo + 256) >> 9);
}

// ALU op 6 SILU32 on one value (gen_layer_script.py:1409-1413).
__device__ __forceinline__ int32_t silu32(int64_t y, int shift, const int32_t *sig) {
  const int64_t x = clamp64(movy_shift(y, shift), -(1 << 20), (1 << 20) - 1);
  const int32_t s = sigmoid_q((int32_t)x, sig);
  return (int32_t)clamp64(rshr64(x * s, 15), -32768, 32767);
}

// 1/sqrt(v * 2^-P) ~= r * 2^(e-30): fixedpoint.py:56-75.
__device__ void rsqrt_q(uint64_t v, int P, const int32_t *lut, int64_t *r_out,
                        int *e_out) {
  const int bl = 64 - __clzll((long long)v);
  int s = bl - 32;
  if ((s - P) & 1) s += 1;
  const int64_t m = (int64_t)(s >= 0 ? (v >> s) : (v << (-s)));
  const int E = s - P + 30;
  const int idx = (m < ((int64_t)1 << 31)) ? (int)((m >> 22) & 0xFF)
                                           : (256 | (int)((m >> 23) & 0xFF));
  int64_t r = (int64_t)lut[idx] << 15;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int64_t r2 = (r * r) >> 30;
    const int64_t mr2 = (m * r2) >> 30;
    r = (r * (((int64_t)3 << 30) - mr2)) >> 31;
  }
  *r_out = r;
  *e_out = -(E / 2);
}

// ---------------------------------------------------------------------------
// workgroup reductions (4 wavefronts of 64)
// ---------------------------------------------------------------------------
// Wavefront reductions on the DPP network: pairs, quads, half rows and
// rows by quad_perm / mirror moves, then rows 0..3 through row_bcast15 and
// row_bcast31; lane 63 ends with the total.  Lanes a row_mask leaves out
// read the identity.
#define W4A8_DPP(v, ident, ctrl, rowmask) \
  __builtin_amdgcn_update_dpp((ident), (v), (ctrl), (rowmask), 0xF, false)

__device__ __forceinline__ int32_t wave_max_i32(int32_t v) {
  // v >= 0 (magnitudes), so 0 is the identity
  v = max(v, W4A8_DPP(v, 0, 0xB1, 0xF));    // quad_perm [1,0,3,2]
  v = max(v, W4A8_DPP(v, 0, 0x4E, 0xF));    // quad_perm [2,3,0,1]
  v = max(v, W4A8_DPP(v, 0, 0x141, 0xF));   // row_half_mirror
  v = max(v, W4A8_DPP(v, 0, 0x140, 0xF));   // row_mirror
  v = max(v, W4A8_DPP(v, 0, 0x142, 0xA));   // row_bcast15 -> rows 1, 3
  v = max(v, W4A8_DPP(v, 0, 0x143, 0xC));   // row_bcast31 -> rows 2, 3
  return __builtin_amdgcn_readlane(v, 63);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL,
                                                            ROWMASK, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32),
                                                            CTRL, ROWMASK, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  v += dpp_u64<0xB1, 0xF>(v);
  v += dpp_u64<0x4E, 0xF>(v);
  v += dpp_u64<0x141, 0xF>(v);
  v += dpp_u64<0x140, 0xF>(v);
  v += dpp_u64<0x142, 0xA>(v);
  v += dpp_u64<0x143, 0xC>(v);
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

__device__ int32_t block_max_i32(int32_t v, int64_t *sm) {
  v = wave_max_i32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = v;
  __syncthreads();
  int32_t r = (int32_t)sm[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = max(r, (int32_t)sm[i]);
  return r;
}
__device__ uint64_t block_sum_u64(uint64_t v, int64_t *sm) {
  v = wave_sum_u64(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = (int64_t)v;
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r += (uint64_t)sm[i];
  return r;
}

// ---------------------------------------------------------------------------
// prologue: produce x8 (and e_x) in LDS.  Every workgroup computes the same
// values (DYNQ8 is one exponent over the whole vector and cannot be chunked,
// SEQ_ISA.md:560-569), so no grid-wide synchronisation is needed.
// ---------------------------------------------------------------------------
constexpr int kPieces = kKMax / (kWG * 8);   // 6 pieces of 8 int16 per thread

__device__ __forceinline__ int16_t piece_get(const int4 &p, int j) {
  const int32_t w = j < 2 ? p.x : (j < 4 ? p.y : (j < 6 ? p.z : p.w));
  return (int16_t)((j & 1) ? (w >> 16) : (w & 0xFFFF));
}
__device__ __forceinline__ void piece_set(int4 &p, int j, int16_t v) {
  int32_t *w = j < 2 ? &p.x : (j < 4 ? &p.y : (j < 6 ? &p.z : &p.w));
  if (j & 1) *w = (int32_t)(((uint32_t)*w & 0xFFFFu) | ((uint32_t)(uint16_t)v << 16));
  else       *w = (int32_t)(((uint32_t)*w & 0xFFFF0000u) | (uint32_t)(uint16_t)v);
}


// The activation vector of one site, held in registers from the moment its
// loads are issued (before any weight load, so it is not queued behind the
// weight stream) until the prologue consumes it.
constexpr int kNormPieces = 8192 / (kWG * 8);   // RMSNorm vectors are <= 8192

struct XRegs {
  int4 pc[kPieces];       // int16 x (or, for PRO_X8, 16 int8 per piece)
  int4 wv[kNormPieces];   // int16 norm weights
};

// Pieces c < npieces(K) hold data; the count is uniform, so the unrolled
// piece loops below branch on scalars and never run masked-off pieces.
__device__ __forceinline__ int npieces(int K, int per_piece) {
  return (K + kWG * per_piece - 1) / (kWG * per_piece);
}

__device__ __forceinline__ void prologue_load(const GemvParams &P, XRegs &X) {
  const int tid = threadIdx.x;
  const int K = P.K;
  if (P.pro == PRO_X8) {
    const int8_t *x = (const int8_t *)P.x;
    const int np = npieces(K, 16);
#pragma unroll
    for (int c = 0; c < kPieces / 2; ++c) {
      if (c < np) {
        const int i = (c * kWG + tid) * 16;
        if (i < K) X.pc[c] = *(const int4 *)(x + i);
      }
    }
    return;
  }
  const int16_t *x16 = (const int16_t *)P.x;
  const int np = npieces(K, 8);
#pragma unroll
  for (int c = 0; c < kPieces; ++c) {
    if (c < np) {
      const int base = c * kWG * 8 + tid * 8;
      X.pc[c] = base < K ? *(const int4 *)(x16 + base) : make_int4(0, 0, 0, 0);
    }
  }
  if (P.pro == PRO_RMSNORM_DYNQ8) {
#pragma unroll
    for (int c = 0; c < kNormPieces; ++c) {
      if (c < np) {
        const int base = c * kWG * 8 + tid * 8;
        X.wv[c] = base < K ? *(const int4 *)(P.norm_w + base) : make_int4(0, 0, 0, 0);
      }
    }
  }
}

// rshift_round of a magnitude (s uniform, >= 0)
__device__ __forceinline__ uint64_t round_shift_mag(uint64_t mag, int s) {
  return s == 0 ? mag : ((mag + ((uint64_t)1 << (s - 1))) >> s);
}

__device__ int prologue_compute(const GemvParams &P, XRegs &X, int8_t *xs, int64_t *sm) {
  const int tid = threadIdx.x;
  const int K = P.K;
  const bool writer = blockIdx.x == 0;
  if (P.pro == PRO_X8) {
    const int np8 = npieces(K, 16);
#pragma unroll
    for (int c = 0; c < kPieces / 2; ++c) {
      const int i = (c * kWG + tid) * 16;
      if (c < np8 && i < K) {
        *(int4 *)(xs + i) = X.pc[c];
        if (writer && P.x8_out) *(int4 *)(P.x8_out + i) = X.pc[c];
      }
    }
    if (writer && P.e_x_out && tid == 0) *P.e_x_out = P.e_x_given;
    return P.e_x_given;
  }
  const int np = npieces(K, 8);
  if (P.pro == PRO_RMSNORM_DYNQ8) {
    // layer_fixed.py:1262-1278, in sign-magnitude form: rshift_round rounds
    // the magnitude, so |x * r| and |y * sc| carry the rounding and the
    // sign is restored afterwards
    uint64_t ss = 0;
#pragma unroll
    for (int c = 0; c < kNormPieces; ++c) {
      if (c < np) {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const int32_t a = piece_get(X.pc[c], j), b = piece_get(X.pc[c], j + 1);
          ss += (uint64_t)((uint32_t)(a * a) + (uint32_t)(b * b));
        }
      }
    }
    ss = block_sum_u64(ss, sm);
    if (ss == 0) ss = 1;
    const int nbits = 31 - __clz(K);
    int64_t r;
    int e;
    rsqrt_q(ss, 2 * P.in_f + nbits, P.tables + kRsqrtOff, &r, &e);
    const int s1 = 30 - e;
    const int32_t one = P.one_plus ? (1 << 14) : 0;
    // |x| * r < 2^46.  Every element step below is branch-free: the right
    // shift (s1 >= 0, capped at 63) and the left shift (s1 < 0) are both
    // formed and the uniform sign of s1 selects one
    const int rs = s1 < 0 ? 0 : (s1 > 63 ? 63 : s1);
    const int ls = s1 < 0 ? (-s1 > 63 ? 63 : -s1) : 0;
    const uint64_t half1 = rs > 0 ? ((uint64_t)1 << (rs - 1)) : 0;
    const bool right = s1 >= 0;
    // pieces past K hold zeros (loaded as such), which normalise to zero:
    // only the stores need the per-thread bound
#pragma unroll
    for (int c = 0; c < kNormPieces; ++c) {
      const int base = c * kWG * 8 + tid * 8;
      if (c < np) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int32_t xv = piece_get(X.pc[c], j);
          const int32_t sc = (int32_t)piece_get(X.wv[c], j) + one;
          const uint64_t mag = (uint64_t)(uint32_t)abs(xv) * (uint64_t)r;
          uint64_t ym = right ? ((mag + half1) >> rs) : (mag << ls);
          // clip to [-2^32, 2^32 - 1]
          const uint64_t cap = (uint64_t)0xFFFFFFFFu + (uint64_t)(xv < 0);
          ym = ym < cap ? ym : cap;
          // rshift_round(y * sc, 14) on the magnitude, then clip16
          const uint64_t q = (ym * (uint64_t)(uint32_t)abs(sc) + 8192u) >> 14;
          const bool neg = (xv < 0) != (sc < 0);
          const int32_t q32 = q > 65535u ? 65535 : (int32_t)q;
          const int32_t qm = min(q32, 32767 + (int32_t)neg);
          piece_set(X.pc[c], j, (int16_t)(neg ? -qm : qm));
        }
        if (writer && P.xn_out && base < K) *(int4 *)(P.xn_out + base) = X.pc[c];
      }
    }
  }
  int32_t mx = 0;
#pragma unroll
  for (int c = 0; c < kPieces; ++c)
    if (c < np)
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = max(mx, abs((int32_t)piece_get(X.pc[c], j)));
  mx = block_max_i32(mx, sm);
  int e = 0;
  while (((mx + ((1 << e) >> 1)) >> e) > 127) ++e;
  const int32_t half = (1 << e) >> 1;
#pragma unroll
  for (int c = 0; c < kPieces; ++c) {
    const int base = c * kWG * 8 + tid * 8;
    if (c < np) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int32_t v = piece_get(X.pc[c], j);
        const int32_t qm = min((abs(v) + half) >> e, 127);
        const uint32_t b = (uint32_t)(uint8_t)(int8_t)(v < 0 ? -qm : qm);
        if (j < 4) lo |= b << (8 * j);
        else       hi |= b << (8 * (j - 4));
      }
      if (base < K) {
        *(uint2 *)(xs + base) = make_uint2(lo, hi);
        if (writer && P.x8_out) *(uint2 *)(P.x8_out + base) = make_uint2(lo, hi);
      }
    }
  }
  if (writer && P.e_x_out && tid == 0) *P.e_x_out = e;
  return e;
}

// ---------------------------------------------------------------------------
// the GEMV
// ---------------------------------------------------------------------------
__device__ __forceinline__ int dot_group(const uint4 &w, const int8_t *xq,
                                         int neg_corr) {
  // 32 weights of one lane against x8[k0 .. k0+32): returns 16 * sum w*x.
  // neg_corr = -8 * (sum of the x8 met by the offset-form low nibbles)
  const int4 xa = *(const int4 *)xq;
  const int4 xb = *(const int4 *)(xq + 16);
  int a = neg_corr, b = 0;
  a = __builtin_amdgcn_sdot4((int)(w.x & 0x0F0F0F0Fu), xa.x, a, false);
  b = __builtin_amdgcn_sdot4((int)(w.x & 0xF0F0F0F0u), xa.y, b, false);
  a = __builtin_amdgcn_sdot4((int)(w.y & 0x0F0F0F0Fu), xa.z, a, false);
  b = __builtin_amdgcn_sdot4((int)(w.y & 0xF0F0F0F0u), xa.w, b, false);
  a = __builtin_amdgcn_sdot4((int)(w.z & 0x0F0F0F0Fu), xb.x, a, false);
  b = __builtin_amdgcn_sdot4((int)(w.z & 0xF0F0F0F0u), xb.y, b, false);
  a = __builtin_amdgcn_sdot4((int)(w.w & 0x0F0F0F0Fu), xb.z, a, false);
  b = __builtin_amdgcn_sdot4((int)(w.w & 0xF0F0F0F0u), xb.w, b, false);
  return (a << 4) + b;
}

__device__ __forceinline__ uint32_t scale_of(const uint4 &sc, int i) {
  const uint32_t w = i < 2 ? sc.x : (i < 4 ? sc.y : (i < 6 ? sc.z : sc.w));
  return (i & 1) ? (w >> 16) : (w & 0xFFFFu);
}

__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return ldg16_nt(p); }

// One scale block (8 groups, fewer in the last block) of one tile, as held
// by one lane: its 16-byte scale row and 8 weight pieces of 32 weights.
struct BlockRegs {
  uint4 sc;
  uint4 w[kGroupsPerBlock];
};

__device__ __forceinline__ void load_block(BlockRegs &R, const uint8_t *bb, int ng,
                                           int lane) {
  R.sc = ldg16(bb + (lane >> 2) * 16);
#pragma unroll
  for (int i = 0; i < kGroupsPerBlock; ++i)
    if (i < ng) R.w[i] = ldg16(bb + kScaleChunk + i * kGroupChunk + lane * 16);
}

__device__ __forceinline__ int64_t dot_block(const BlockRegs &R, int ng, int g0, int q,
                                             const int8_t *xs, const int32_t *xlo,
                                             int64_t p) {
#pragma unroll
  for (int i = 0; i < kGroupsPerBlock; ++i) {
    if (i < ng) {
      const int g = g0 + i;
      const int s16 = dot_group(R.w[i], xs + kGroup * g + 32 * q, xlo[g * 4 + q]);
      p += (int64_t)(int32_t)scale_of(R.sc, i) * (int64_t)s16;
    }
  }
  return p;
}

__device__ __forceinline__ int job_of(const GemvParams &P, int tg) {
  // unrolled over the fixed job table so every tile0 is loaded at once
  int j = 0;
#pragma unroll
  for (int k = 1; k < kMaxJobs; ++k) j += (k < P.njobs && tg >= P.job[k].tile0) ? 1 : 0;
  return j;
}

__device__ __forceinline__ const uint8_t *block_addr(const GemvParams &P, int tg, int b) {
  const int j = job_of(P, tg);
  return P.job[j].w + (int64_t)(tg - P.job[j].tile0) * P.tile_bytes +
         (int64_t)b * kBlockBytes;
}

__device__ __forceinline__ int groups_in(int NG, int b) {
  return min(kGroupsPerBlock, NG - b * kGroupsPerBlock);
}

// x8 in LDS -> -8 * sum of the x8 values that meet the offset-form low
// nibbles of each (group, quarter): dwords 0,2,4,6 of every 32-byte piece
__device__ __forceinline__ void build_corrections(const int8_t *xs, int32_t *xlo, int NG) {
  for (int c = threadIdx.x; c < NG * 4; c += kWG) {
    const int *xw = (const int *)(xs + 32 * c);
    int s = 0;
    s = __builtin_amdgcn_sdot4(xw[0], 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(xw[2], 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(xw[4], 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(xw[6], 0x01010101, s, false);
    xlo[c] = -8 * s;
  }
}

__device__ __forceinline__ uint64_t argmax_key(int32_t v, uint32_t row) {
  return ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | (uint64_t)(0xFFFFFFFFu - row);
}

// reduce a tile's 16 * p over the 4 k-quarter lanes and the 4 wavefronts,
// then round, check and write the 16 rows (one wavefront, rotating per tile)
__device__ __forceinline__ void tile_finish(const GemvJob &J, int t, int64_t p, int it,
                                            int wave, int lane, int e_x,
                                            const int32_t *sig, int32_t *err,
                                            int64_t (*red)[kWaves][kTileRows],
                                            uint64_t &best) {
  // sum the 4 k-quarter lanes of each row (lanes 4r..4r+3: one DPP quad)
  p = (int64_t)((uint64_t)p + dpp_u64<0xB1, 0xF>((uint64_t)p));
  p = (int64_t)((uint64_t)p + dpp_u64<0x4E, 0xF>((uint64_t)p));
  const int par = it & 1;
  if ((lane & 3) == 0) red[par][wave][lane >> 2] = p;
  __syncthreads();
  if (wave == (it & (kWaves - 1)) && lane < kTileRows) {
    int64_t tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += red[par][w][lane];
    const int row = t * kTileRows + lane;
    if (row < J.nrows) {
      const int64_t y = rshr64(tot >> 4, J.sh);   // tot is 16 * p exactly
      if (y > 2147483647LL || y < -2147483647LL) atomicOr(err, 1);
      const int shift = J.p0 - e_x;
      switch (J.epi) {
        case EPI_Y32:
          ((int32_t *)J.out)[row] = (int32_t)y;
          break;
        case EPI_MOVY_I16:
          ((int16_t *)J.out)[row] = (int16_t)clamp64(movy_shift(y, shift), -32768, 32767);
          break;
        case EPI_MOVY_P32:
          ((int32_t *)J.out)[row] =
              (int32_t)clamp64(movy_shift(y, shift), -2147483648LL, 2147483647LL);
          break;
        case EPI_SILU32:
          ((int16_t *)J.out)[row] = (int16_t)silu32(y, shift, sig);
          break;
        case EPI_SHIFT_I64:
          ((int64_t *)J.out)[row] = movy_shift(y, shift);
          break;
        default: {   // EPI_ARGMAX: raw y32 (shift 0), seq_format.py:2225-2226
          const uint64_t k = argmax_key((int32_t)y, (uint32_t)row);
          best = k > best ? k : best;
        }
      }
    }
  }
}

__device__ __forceinline__ void write_partial(uint64_t best, uint64_t *partials,
                                              uint64_t *keys, int wave, int lane) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t other = __shfl_xor(best, o);
    best = other > best ? other : best;
  }
  __syncthreads();
  if (lane == 0) keys[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t k = keys[0];
    for (int w = 1; w < kWaves; ++w) k = keys[w] > k ? keys[w] : k;
    partials[blockIdx.x] = k;
  }
}

__global__ __launch_bounds__(kWG) void gemv_kernel(GemvParams P) {
  __shared__ __align__(16) int8_t xs[kKMax];
  __shared__ int32_t xlo[kKMax / 32];
  __shared__ int64_t red[2][kWaves][kTileRows];
  __shared__ int64_t sm[kWaves];
  __shared__ uint64_t keys[kWaves];

  const int tid = threadIdx.x, lane = tid & 63, q = lane & 3;
  // wave index as a scalar so the block loop below branches on SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NG = P.NG, nblk = P.nblk;
  // The activation loads go out first; the weights do not depend on x, so
  // this wave's first block is put in flight right behind them and both
  // memory latencies overlap with the prologue.
  XRegs X;
  prologue_load(P, X);
  BlockRegs cur;
  if ((int)blockIdx.x < P.total_tiles && wave < nblk)
    load_block(cur, block_addr(P, blockIdx.x, wave), groups_in(NG, wave), lane);
  const int e_x = prologue_compute(P, X, xs, sm);
  __syncthreads();
  build_corrections(xs, xlo, NG);
  __syncthreads();

  const int32_t *sig = P.tables + kSigmoidOff;
  uint64_t best = 0;   // argmax key (0 == none)
  int it = 0;
  for (int tg = blockIdx.x; tg < P.total_tiles; tg += gridDim.x, ++it) {
    const GemvJob &J = P.job[job_of(P, tg)];
    const int t = tg - J.tile0;
    int64_t p = 0;
    for (int b = wave; b < nblk; b += kWaves) {
      // prefetch this wave's next block (same tile, or its next tile)
      int nb = b + kWaves, ntg = tg;
      if (nb >= nblk) {
        nb = wave;
        ntg = tg + gridDim.x;
      }
      const bool more = ntg < P.total_tiles;
      BlockRegs nxt;
      if (more) load_block(nxt, block_addr(P, ntg, nb), groups_in(NG, nb), lane);
      p = dot_block(cur, groups_in(NG, b), b * kGroupsPerBlock, q, xs, xlo, p);
      if (more) cur = nxt;
    }
    tile_finish(J, t, p, it, wave, lane, e_x, sig, P.err, red, best);
  }
  if (P.partials) write_partial(best, P.partials, keys, wave, lane);
}

// ---------------------------------------------------------------------------
// persistent decode-step kernel
//
// One cooperative launch runs every site of a plan, one 512-thread
// workgroup per CU: two teams of four wavefronts.  Team v (of V = 2G) takes
// tiles (v + tile_rot) mod V, + V, ... of each site; its four wavefronts
// split a tile's scale blocks.  Site s+1 starts only after all G workgroups
// have finished site s -- the dependency a decode step has between
// consecutive DYNQ8 sites -- counted per XCD, then globally.  The data that
// crosses that dependency travels with agent-coherent accesses: outputs are
// stored and activation vectors loaded with device-scope atomics, so the
// ordering needs no cache-wide writeback or invalidation.  Weights never
// depend on an activation, so each wavefront keeps its next weight block in
// flight across the wait.
// ---------------------------------------------------------------------------
constexpr int kSWG = 512;                 // threads per stream workgroup
constexpr int kSWaves = kSWG / 64;        // 8
constexpr int kTeams = kStreamTeams;      // 2 teams of 4 wavefronts
static_assert(kSWaves == 4 * kTeams, "a team is 4 wavefronts");
constexpr int kSPieces = kKMax / (kSWG * 8);       // 3 pieces of 8 x per thread
constexpr int kSNormPieces = 8192 / (kSWG * 8);    // 2
constexpr uint32_t kSpinLimit = 1u << 18;          // a wait that never ends
                                                   // flags err bit 1, moves on
constexpr int kXcds = 8;
constexpr int kCounterStride = 64;                 // uint32 words: 256 B apart

struct SRegs {
  int4 pc[kSPieces];
  int4 wv[kSNormPieces];
};

__device__ __forceinline__ int4 load_coherent16(const void *p) {
  const uint64_t *q = (const uint64_t *)p;
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_int4((int)(uint32_t)a, (int)(uint32_t)(a >> 32), (int)(uint32_t)b,
                   (int)(uint32_t)(b >> 32));
}

template <typename T>
__device__ __forceinline__ void store_coherent(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int32_t sblock_max(int32_t v, int64_t *sm) {
  v = wave_max_i32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = v;
  __syncthreads();
  int32_t r = (int32_t)sm[0];
#pragma unroll
  for (int i = 1; i < kSWaves; ++i) r = max(r, (int32_t)sm[i]);
  return r;
}
__device__ __forceinline__ uint64_t sblock_sum(uint64_t v, int64_t *sm) {
  v = wave_sum_u64(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = (int64_t)v;
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < kSWaves; ++i) r += (uint64_t)sm[i];
  return r;
}

// the site's activation vector -> x8 in LDS (512 threads, coherent loads)
__device__ int stream_prologue(const GemvParams &P, int8_t *xs, int64_t *sm) {
  const int tid = threadIdx.x;
  const int K = P.K;
  const bool writer = blockIdx.x == 0;
  SRegs X;
  if (P.pro == PRO_X8) {
    for (int i = tid * 16; i < K; i += kSWG * 16) {
      const int4 v = load_coherent16((const int8_t *)P.x + i);
      *(int4 *)(xs + i) = v;
      if (writer && P.x8_out) *(int4 *)(P.x8_out + i) = v;
    }
    if (writer && P.e_x_out && tid == 0) *P.e_x_out = P.e_x_given;
    return P.e_x_given;
  }
  const int np = (K + kSWG * 8 - 1) / (kSWG * 8);
  const int16_t *x16 = (const int16_t *)P.x;
#pragma unroll
  for (int c = 0; c < kSPieces; ++c) {
    if (c < np) {
      const int base = c * kSWG * 8 + tid * 8;
      X.pc[c] = base < K ? load_coherent16(x16 + base) : make_int4(0, 0, 0, 0);
    }
  }
  if (P.pro == PRO_RMSNORM_DYNQ8) {
#pragma unroll
    for (int c = 0; c < kSNormPieces; ++c) {
      if (c < np) {
        const int base = c * kSWG * 8 + tid * 8;
        X.wv[c] = base < K ? *(const int4 *)(P.norm_w + base) : make_int4(0, 0, 0, 0);
      }
    }
    uint64_t ss = 0;
#pragma unroll
    for (int c = 0; c < kSNormPieces; ++c)
      if (c < np)
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const int32_t a = piece_get(X.pc[c], j), b2 = piece_get(X.pc[c], j + 1);
          ss += (uint64_t)((uint32_t)(a * a) + (uint32_t)(b2 * b2));
        }
    ss = sblock_sum(ss, sm);
    if (ss == 0) ss = 1;
    int64_t r;
    int e;
    rsqrt_q(ss, 2 * P.in_f + (31 - __clz(K)), P.tables + kRsqrtOff, &r, &e);
    const int s1 = 30 - e;
    const int32_t one = P.one_plus ? (1 << 14) : 0;
    const int rs = s1 < 0 ? 0 : (s1 > 63 ? 63 : s1);
    const int ls = s1 < 0 ? (-s1 > 63 ? 63 : -s1) : 0;
    const uint64_t half1 = rs > 0 ? ((uint64_t)1 << (rs - 1)) : 0;
    const bool right = s1 >= 0;
#pragma unroll
    for (int c = 0; c < kSNormPieces; ++c) {
      const int base = c * kSWG * 8 + tid * 8;
      if (c < np) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int32_t xv = piece_get(X.pc[c], j);
          const int32_t sc = (int32_t)piece_get(X.wv[c], j) + one;
          const uint64_t mag = (uint64_t)(uint32_t)abs(xv) * (uint64_t)r;
          uint64_t ym = right ? ((mag + half1) >> rs) : (mag << ls);
          const uint64_t cap = (uint64_t)0xFFFFFFFFu + (uint64_t)(xv < 0);
          ym = ym < cap ? ym : cap;
          const uint64_t q = (ym * (uint64_t)(uint32_t)abs(sc) + 8192u) >> 14;
          const bool neg = (xv < 0) != (sc < 0);
          const int32_t q32 = q > 65535u ? 65535 : (int32_t)q;
          const int32_t qm = min(q32, 32767 + (int32_t)neg);
          piece_set(X.pc[c], j, (int16_t)(neg ? -qm : qm));
        }
        if (writer && P.xn_out && base < K) *(int4 *)(P.xn_out + base) = X.pc[c];
      }
    }
  }
  int32_t mx = 0;
#pragma unroll
  for (int c = 0; c < kSPieces; ++c)
    if (c < np)
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = max(mx, abs((int32_t)piece_get(X.pc[c], j)));
  mx = sblock_max(mx, sm);
  int e = 0;
  while (((mx + ((1 << e) >> 1)) >> e) > 127) ++e;
  const int32_t half = (1 << e) >> 1;
#pragma unroll
  for (int c = 0; c < kSPieces; ++c) {
    const int base = c * kSWG * 8 + tid * 8;
    if (c < np) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int32_t v = piece_get(X.pc[c], j);
        const int32_t qm = min((abs(v) + half) >> e, 127);
        const uint32_t b8 = (uint32_t)(uint8_t)(int8_t)(v < 0 ? -qm : qm);
        if (j < 4) lo |= b8 << (8 * j);
        else       hi |= b8 << (8 * (j - 4));
      }
      if (base < K) {
        *(uint2 *)(xs + base) = make_uint2(lo, hi);
        if (writer && P.x8_out) *(uint2 *)(P.x8_out + base) = make_uint2(lo, hi);
      }
    }
  }
  if (writer && P.e_x_out && tid == 0) *P.e_x_out = e;
  return e;
}

__device__ __forceinline__ void sbuild_corrections(const int8_t *xs, int32_t *xlo, int NG) {
  for (int c = threadIdx.x; c < NG * 4; c += kSWG) {
    const int *xw = (const int *)(xs + 32 * c);
    int t = 0;
    t = __builtin_amdgcn_sdot4(xw[0], 0x01010101, t, false);
    t = __builtin_amdgcn_sdot4(xw[2], 0x01010101, t, false);
    t = __builtin_amdgcn_sdot4(xw[4], 0x01010101, t, false);
    t = __builtin_amdgcn_sdot4(xw[6], 0x01010101, t, false);
    xlo[c] = -8 * t;
  }
}

// first tile of team v (of V) in a site
__device__ __forceinline__ int team_first(const GemvParams &P, int v, int V) {
  return (v + P.tile_rot) % V;
}

// next (site, tile, block) of wavefront wt of team v after (s, t, b)
__device__ __forceinline__ void snext(const StreamParams &S, int s, int t, int b, int v,
                                      int V, int wt, int &ns, int &nt, int &nb) {
  const GemvParams &P = S.sites[s];
  if (b + 4 < P.nblk) {
    ns = s; nt = t; nb = b + 4;
    return;
  }
  if (t + V < P.total_tiles) {
    ns = s; nt = t + V; nb = wt;
    return;
  }
  for (int s2 = s + 1; s2 < S.nsites; ++s2) {
    const GemvParams &Q = S.sites[s2];
    const int t0 = team_first(Q, v, V);
    if (t0 < Q.total_tiles && wt < Q.nblk) {
      ns = s2; nt = t0; nb = wt;
      return;
    }
  }
  ns = -1; nt = 0; nb = 0;
}

// this workgroup's stores are complete and counted: per XCD, then, by the
// XCD's last workgroup, globally
__device__ __forceinline__ void site_arrive(uint32_t *cnt) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int xcd = blockIdx.x % kXcds;
    const uint32_t per = (gridDim.x - xcd + kXcds - 1) / kXcds;
    const uint32_t old = __hip_atomic_fetch_add(cnt + kCounterStride * (1 + xcd), 1u,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1 == per)
      __hip_atomic_fetch_add(cnt, per, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ __forceinline__ void site_wait(const uint32_t *cnt, uint32_t target,
                                          int32_t *err) {
  if (threadIdx.x == 0) {
    uint32_t n = 0;
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(1);
      if (++n > kSpinLimit) {
        atomicOr(err, 2);
        break;
      }
    }
  }
  __syncthreads();
}

// as tile_finish, for a team of the stream workgroup; outputs are stored
// coherently (they cross the site dependency)
__device__ __forceinline__ void sfinish(const GemvJob &J, int t, bool valid, int64_t p,
                                        int it, int team, int wt, int lane, int e_x,
                                        const int32_t *sig, int32_t *err,
                                        int64_t (*red)[kTeams][4][kTileRows],
                                        uint64_t &best) {
  p = (int64_t)((uint64_t)p + dpp_u64<0xB1, 0xF>((uint64_t)p));
  p = (int64_t)((uint64_t)p + dpp_u64<0x4E, 0xF>((uint64_t)p));
  const int par = it & 1;
  if ((lane & 3) == 0) red[par][team][wt][lane >> 2] = p;
  __syncthreads();
  if (valid && wt == (it & 3) && lane < kTileRows) {
    const int64_t tot = red[par][team][0][lane] + red[par][team][1][lane] +
                        red[par][team][2][lane] + red[par][team][3][lane];
    const int row = t * kTileRows + lane;
    if (row < J.nrows) {
      const int64_t y = rshr64(tot >> 4, J.sh);
      if (y > 2147483647LL || y < -2147483647LL) atomicOr(err, 1);
      const int shift = J.p0 - e_x;
      switch (J.epi) {
        case EPI_Y32:
          store_coherent((int32_t *)J.out + row, (int32_t)y);
          break;
        case EPI_MOVY_I16:
          store_coherent((int16_t *)J.out + row,
                         (int16_t)clamp64(movy_shift(y, shift), -32768, 32767));
          break;
        case EPI_MOVY_P32:
          store_coherent((int32_t *)J.out + row,
                         (int32_t)clamp64(movy_shift(y, shift), -2147483648LL, 2147483647LL));
          break;
        case EPI_SILU32:
          store_coherent((int16_t *)J.out + row, (int16_t)silu32(y, shift, sig));
          break;
        case EPI_SHIFT_I64:
          store_coherent((int64_t *)J.out + row, movy_shift(y, shift));
          break;
        default: {
          const uint64_t k = argmax_key((int32_t)y, (uint32_t)row);
          best = k > best ? k : best;
        }
      }
    }
  }
}

__global__ __launch_bounds__(kSWG) void stream_kernel(StreamParams S) {
  __shared__ __align__(16) int8_t xs[kKMax];
  __shared__ int32_t xlo[kKMax / 32];
  __shared__ int64_t red[2][kTeams][4][kTileRows];
  __shared__ int64_t sm[kSWaves];
  __shared__ uint64_t keys[kSWaves];

  const int tid = threadIdx.x, lane = tid & 63, q = lane & 3;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int team = wave >> 2, wt = wave & 3;
  const int G = gridDim.x, V = G * kTeams;
  const int v = blockIdx.x * kTeams + team;

  // the wavefront's pending item and its registers
  int cs = -1, ct = 0, cb = 0;
  for (int s2 = 0; s2 < S.nsites && cs < 0; ++s2) {
    const GemvParams &Q = S.sites[s2];
    const int t0 = team_first(Q, v, V);
    if (t0 < Q.total_tiles && wt < Q.nblk) {
      cs = s2; ct = t0; cb = wt;
    }
  }
  BlockRegs cur;
  if (cs >= 0)
    load_block(cur, block_addr(S.sites[cs], ct, cb), groups_in(S.sites[cs].NG, cb), lane);

  uint64_t best = 0;
  int it = 0;
  for (int s = 0; s < S.nsites; ++s) {
    const GemvParams &P = S.sites[s];
    if (s > 0) site_wait(S.done + kCounterStride * (kXcds + 1) * (s - 1), (uint32_t)G, S.err);
    if (S.trace && blockIdx.x == 0 && tid == 0) S.trace[s] = wall_clock64();
    const int e_x = stream_prologue(P, xs, sm);
    __syncthreads();
    sbuild_corrections(xs, xlo, P.NG);
    __syncthreads();
    const int32_t *sig = P.tables + kSigmoidOff;
    const int first = team_first(P, v, V);
    // every team runs the same number of iterations (the barriers inside
    // are workgroup-wide); a team past its last tile idles through them
    const int iters = (P.total_tiles + V - 1) / V;
    for (int i = 0; i < iters; ++i, ++it) {
      const int t = first + i * V;
      const bool valid = t < P.total_tiles;
      const GemvJob &J = P.job[job_of(P, valid ? t : 0)];
      int64_t p = 0;
      if (valid) {
        for (int b = wt; b < P.nblk; b += 4) {
          int ns, nt, nb;
          snext(S, s, t, b, v, V, wt, ns, nt, nb);
          BlockRegs nxt;
          if (ns >= 0)
            load_block(nxt, block_addr(S.sites[ns], nt, nb), groups_in(S.sites[ns].NG, nb), lane);
          p = dot_block(cur, groups_in(P.NG, b), b * kGroupsPerBlock, q, xs, xlo, p);
          if (ns >= 0) cur = nxt;
        }
      }
      sfinish(J, valid ? t - J.tile0 : 0, valid, p, it, team, wt, lane, e_x, sig, S.err,
              red, best);
    }
    site_arrive(S.done + kCounterStride * (kXcds + 1) * s);
  }
  if (S.trace && blockIdx.x == 0 && tid == 0) S.trace[S.nsites] = wall_clock64();
  if (S.head_site >= 0) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = __shfl_xor(best, o);
      best = other > best ? other : best;
    }
    __syncthreads();
    if (lane == 0) keys[wave] = best;
    __syncthreads();
    if (tid == 0) {
      uint64_t k = keys[0];
      for (int w = 1; w < kSWaves; ++w) k = keys[w] > k ? keys[w] : k;
      S.partials[blockIdx.x] = k;
    }
  }
}

__global__ __launch_bounds__(kWG) void argmax_final_kernel(
    const uint64_t *partials, int n, int32_t *result) {
  __shared__ uint64_t keys[kWaves];
  uint64_t best = 0;
  for (int i = threadIdx.x; i < n; i += kWG) best = partials[i] > best ? partials[i] : best;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t other = __shfl_xor(best, o);
    best = other > best ? other : best;
  }
  if ((threadIdx.x & 63) == 0) keys[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWaves; ++w) best = keys[w] > best ? keys[w] : best;
    best = keys[0] > best ? keys[0] : best;
    result[0] = (int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
    result[1] = (int32_t)((uint32_t)(best >> 32) ^ 0x80000000u);
  }
}

// prologue only: DYNQ8 / RMSNorm(+DYNQ8) of one vector, one workgroup
__global__ __launch_bounds__(kWG) void vec_prologue_kernel(GemvParams P) {
  __shared__ __align__(16) int8_t xs[kKMax];
  __shared__ int64_t sm[kWaves];
  XRegs X;
  prologue_load(P, X);
  prologue_compute(P, X, xs, sm);
}

// ---------------------------------------------------------------------------
// repack: row image (w4a8_ref.py:349-370) <-> tile layout
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t to_tile_word(uint32_t in) {
  // nibble t of `in` is w[k0+t] (two's complement)
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = ((in >> (4 * i)) & 15u) ^ 8u;
    const uint32_t hi = (in >> (4 * (4 + i))) & 15u;
    out |= (lo | (hi << 4)) << (8 * i);
  }
  return out;
}
__device__ __forceinline__ uint32_t from_tile_word(uint32_t out) {
  uint32_t in = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t byte = (out >> (8 * i)) & 0xFFu;
    in |= ((byte & 15u) ^ 8u) << (4 * i);
    in |= (byte >> 4) << (4 * (4 + i));
  }
  return in;
}

__device__ __forceinline__ uint8_t *group_piece(uint8_t *base, const Layout &L,
                                                int64_t r, int g) {
  const int64_t t = r / kTileRows;
  const int rr = (int)(r % kTileRows);
  return base + t * L.tile_bytes + (int64_t)(g / kGroupsPerBlock) * kBlockBytes +
         kScaleChunk + (g % kGroupsPerBlock) * kGroupChunk + rr * 64;
}
__device__ __forceinline__ uint8_t *scale_piece(uint8_t *base, const Layout &L,
                                                int64_t r, int b) {
  const int64_t t = r / kTileRows;
  const int rr = (int)(r % kTileRows);
  return base + t * L.tile_bytes + (int64_t)b * kBlockBytes + rr * 16;
}

__global__ void repack_groups_kernel(const uint8_t *img, int64_t nrows, Layout L,
                                     int64_t stride, uint8_t *dst) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= nrows * L.NG) return;
  const int64_t r = gid / L.NG;
  const int g = (int)(gid % L.NG);
  const uint4 *src = (const uint4 *)(img + r * stride + 64 * g);
  uint4 *d = (uint4 *)group_piece(dst, L, r, g);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 v = src[q];
    d[q] = make_uint4(to_tile_word(v.x), to_tile_word(v.y), to_tile_word(v.z),
                      to_tile_word(v.w));
  }
}

__global__ void repack_scales_kernel(const uint8_t *img, int64_t nrows, Layout L,
                                     int64_t stride, uint8_t *dst) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= nrows * L.nblk) return;
  const int64_t r = gid / L.nblk;
  const int b = (int)(gid % L.nblk);
  const uint8_t *s = img + r * stride + L.K / 2;
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int g = b * kGroupsPerBlock + j;
    if (g < L.NG) {
      const uint32_t m = (uint32_t)s[2 * g] | ((uint32_t)s[2 * g + 1] << 8);
      w[j >> 1] |= m << (16 * (j & 1));
    }
  }
  *(uint4 *)scale_piece(dst, L, r, b) = make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ void unpack_groups_kernel(const uint8_t *src, int64_t nrows, Layout L,
                                     int64_t stride, uint8_t *img) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= nrows * L.NG) return;
  const int64_t r = gid / L.NG;
  const int g = (int)(gid % L.NG);
  const uint4 *s = (const uint4 *)group_piece(const_cast<uint8_t *>(src), L, r, g);
  uint4 *d = (uint4 *)(img + r * stride + 64 * g);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 v = s[q];
    d[q] = make_uint4(from_tile_word(v.x), from_tile_word(v.y),
                      from_tile_word(v.z), from_tile_word(v.w));
  }
}

__global__ void unpack_scales_kernel(const uint8_t *src, int64_t nrows, Layout L,
                                     int64_t stride, uint8_t *img) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= nrows * L.nblk) return;
  const int64_t r = gid / L.nblk;
  const int b = (int)(gid % L.nblk);
  const uint4 v = *(const uint4 *)scale_piece(const_cast<uint8_t *>(src), L, r, b);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint8_t *s = img + r * stride + L.K / 2;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int g = b * kGroupsPerBlock + j;
    if (g < L.NG) {
      const uint32_t m = (w[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
      s[2 * g] = (uint8_t)(m & 0xFF);
      s[2 * g + 1] = (uint8_t)(m >> 8);
    }
  }
}

// ---------------------------------------------------------------------------
// elementwise law ops
// ---------------------------------------------------------------------------
__global__ void fill_i32_kernel(int32_t *p, int32_t v, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void rshift_round_kernel(const int64_t *v, int64_t n, int s, int64_t *out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = rshr64(v[i], s);
}

__global__ void movy_kernel(const int32_t *y, int64_t n, int shift, int mode, void *out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = movy_shift(y[i], shift);
    if (mode == 1) ((int16_t *)out)[i] = (int16_t)clamp64(v, -32768, 32767);
    else ((int32_t *)out)[i] = (int32_t)clamp64(v, -2147483648LL, 2147483647LL);
  }
}

__global__ void alu_kernel(int op, const int32_t *y, const int16_t *b, int64_t n,
                           int p0, const int32_t *tables, void *out) {
  const int32_t *sig = tables + kSigmoidOff;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = y[i];
    switch (op) {
      case 1:   // SHIFT32
        ((int16_t *)out)[i] = (int16_t)clamp64(movy_shift(v, p0), -32768, 32767);
        break;
      case 6:   // SILU32
        ((int16_t *)out)[i] = (int16_t)silu32(v, p0, sig);
        break;
      case 8:   // EMUL32: clip16(rshift_round(y * b, p0))
        ((int16_t *)out)[i] = (int16_t)clamp64(movy_shift(v * (int64_t)b[i], p0),
                                               -32768, 32767);
        break;
      default:  // 9 SHIFT32W
        ((int32_t *)out)[i] = (int32_t)clamp64(movy_shift(v, p0),
                                               -2147483648LL, 2147483647LL);
    }
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static int blocks_for(int64_t n, int threads, int cap) {
  int64_t b = (n + threads - 1) / threads;
  if (b < 1) b = 1;
  return (int)(b > cap ? cap : b);
}

hipError_t launch_fill_i32(int32_t *p, int32_t v, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks_for(n, 256, 4096)), dim3(256),
                     0, s, p, v, n);
  return hipGetLastError();
}

hipError_t launch_repack(const uint8_t *img, int64_t nrows, const Layout &L,
                         int64_t stride, uint8_t *dst, hipStream_t s) {
  const int64_t ntiles = (nrows + kTileRows - 1) / kTileRows;
  hipError_t e = hipMemsetAsync(dst, 0, (size_t)(ntiles * L.tile_bytes), s);
  if (e != hipSuccess) return e;
  const int64_t ng = nrows * L.NG, nb = nrows * L.nblk;
  hipLaunchKernelGGL(repack_groups_kernel, dim3((unsigned)((ng + 255) / 256)),
                     dim3(256), 0, s, img, nrows, L, stride, dst);
  hipLaunchKernelGGL(repack_scales_kernel, dim3((unsigned)((nb + 255) / 256)),
                     dim3(256), 0, s, img, nrows, L, stride, dst);
  return hipGetLastError();
}

hipError_t launch_unpack(const uint8_t *src, int64_t nrows, const Layout &L,
                         int64_t stride, uint8_t *img, hipStream_t s) {
  hipError_t e = hipMemsetAsync(img, 0, (size_t)(nrows * stride), s);
  if (e != hipSuccess) return e;
  const int64_t ng = nrows * L.NG, nb = nrows * L.nblk;
  hipLaunchKernelGGL(unpack_groups_kernel, dim3((unsigned)((ng + 255) / 256)),
                     dim3(256), 0, s, src, nrows, L, stride, img);
  hipLaunchKernelGGL(unpack_scales_kernel, dim3((unsigned)((nb + 255) / 256)),
                     dim3(256), 0, s, src, nrows, L, stride, img);
  return hipGetLastError();
}

hipError_t launch_gemv(const GemvParams &p, int grid, hipStream_t s) {
  hipLaunchKernelGGL(gemv_kernel, dim3(grid), dim3(kWG), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_gemv_timed(const GemvParams &p, int grid, hipStream_t s,
                             hipEvent_t start, hipEvent_t stop) {
  hipExtLaunchKernelGGL(gemv_kernel, dim3(grid), dim3(kWG), 0, s, start, stop, 0, p);
  return hipGetLastError();
}

hipError_t launch_argmax_final(const uint64_t *partials, int n, int32_t *result,
                               hipStream_t s) {
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kWG), 0, s, partials, n,
                     result);
  return hipGetLastError();
}

hipError_t launch_vec_prologue(const GemvParams &p, hipStream_t s) {
  hipLaunchKernelGGL(vec_prologue_kernel, dim3(1), dim3(kWG), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_rshift_round(const int64_t *v, int64_t n, int sft, int64_t *out,
                               hipStream_t s) {
  hipLaunchKernelGGL(rshift_round_kernel, dim3(blocks_for(n, 256, 4096)), dim3(256),
                     0, s, v, n, sft, out);
  return hipGetLastError();
}

hipError_t launch_movy(const int32_t *y, int64_t n, int shift, int mode, void *out,
                       hipStream_t s) {
  hipLaunchKernelGGL(movy_kernel, dim3(blocks_for(n, 256, 4096)), dim3(256), 0, s,
                     y, n, shift, mode, out);
  return hipGetLastError();
}

hipError_t launch_alu(int op, const int32_t *y, const int16_t *b, int64_t n, int p0,
                      const int32_t *tables, void *out, hipStream_t s) {
  hipLaunchKernelGGL(alu_kernel, dim3(blocks_for(n, 256, 4096)), dim3(256), 0, s,
                     op, y, b, n, p0, tables, out);
  return hipGetLastError();
}

hipError_t launch_stream(const StreamParams &sp, int grid, hipStream_t s) {
  void *args[] = {(void *)&sp};
  return hipLaunchCooperativeKernel((const void *)stream_kernel, dim3(grid), dim3(kSWG),
                                    args, 0, s);
}

int stream_max_blocks_per_cu() { return 1; }

size_t stream_counter_words(int nsites) {
  return (size_t)kCounterStride * (kXcds + 1) * (size_t)nsites;
}

int gemv_max_blocks_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_kernel, kWG, 0) !=
          hipSuccess || n < 1)
    n = 4;
  return n;
}

}  // namespace w4a8
