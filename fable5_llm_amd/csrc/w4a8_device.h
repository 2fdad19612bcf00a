// Device helpers shared by the GEMV kernels (w4a8_kernels.hip) and the
// persistent stream kernel (w4a8_stream.hip): the integer law's scalar
// steps, DPP wavefront reductions, and the tile-layout dot product.
#pragma once
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
template <typename T>
__device__ __forceinline__ int32_t sigmoid_q(int32_t x, const T *tab) {
  x = x < -(16 << 12) ? -(16 << 12) : (x > (16 << 12) - 1 ? (16 << 12) - 1 : x);
  const int32_t u = x + (16 << 12);
  const int32_t i = u >> 9, lo = u & 0x1FF;
  const int32_t a = (int32_t)tab[i], b = (int32_t)tab[i + 1];
  return a + (((b - a) * lo + 256) >> 9);
}

// ALU op 6 SILU32 on one value (gen_layer_script.py:1409-1413).
template <typename T>
__device__ __forceinline__ int32_t silu32(int64_t y, int shift, const T *sig) {
  const int64_t x = clamp64(movy_shift(y, shift), -(1 << 20), (1 << 20) - 1);
  const int32_t s = sigmoid_q((int32_t)x, sig);
  return (int32_t)clamp64(rshr64(x * s, 15), -32768, 32767);
}

// 1/sqrt(v * 2^-P) ~= r * 2^(e-30): fixedpoint.py:56-75.
template <typename T>
__device__ void rsqrt_q(uint64_t v, int P, const T *lut, int64_t *r_out, int *e_out) {
  const int bl = 64 - __clzll((long long)v);
  int s = bl - 32;
  if ((s - P) & 1) s += 1;
  const int64_t m = (int64_t)(s >= 0 ? (v >> s) : (v << (-s)));
  const int E = s - P + 30;
  const int idx = (m < ((int64_t)1 << 31)) ? (int)((m >> 22) & 0xFF)
                                           : (256 | (int)((m >> 23) & 0xFF));
  int64_t r = (int64_t)(int32_t)lut[idx] << 15;
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

__device__ __forceinline__ int16_t piece_get(const int4 &p, int j) {
  const int32_t w = j < 2 ? p.x : (j < 4 ? p.y : (j < 6 ? p.z : p.w));
  return (int16_t)((j & 1) ? (w >> 16) : (w & 0xFFFF));
}
__device__ __forceinline__ void piece_set(int4 &p, int j, int16_t v) {
  int32_t *w = j < 2 ? &p.x : (j < 4 ? &p.y : (j < 6 ? &p.z : &p.w));
  if (j & 1) *w = (int32_t)(((uint32_t)*w & 0xFFFFu) | ((uint32_t)(uint16_t)v << 16));
  else       *w = (int32_t)(((uint32_t)*w & 0xFFFF0000u) | (uint32_t)(uint16_t)v);
}

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

template <typename PT>
__device__ __forceinline__ int job_of(const PT &P, int tg) {
  // unrolled over the fixed table of first tiles, so they load at once
  int j = 0;
#pragma unroll
  for (int k = 1; k < kMaxJobs; ++k) j += (k < P.njobs && tg >= P.tile0[k]) ? 1 : 0;
  return j;
}

__device__ __forceinline__ int groups_in(int NG, int b) {
  return min(kGroupsPerBlock, NG - b * kGroupsPerBlock);
}

__device__ __forceinline__ uint64_t argmax_key(int32_t v, uint32_t row) {
  return ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | (uint64_t)(0xFFFFFFFFu - row);
}

__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return ldg16_nt(p); }

// ---------------------------------------------------------------------------
// LDS flags between wavefronts.  Written as inline assembly: the compiler's
// own LDS synchronisation (workgroup fences, __syncthreads) also waits for
// every outstanding global load of the wavefront.  A wavefront's LDS
// instructions execute in order, so a flag written after data is seen after
// it, and data read after a flag was seen is current.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t lds_off(const void *p) {
  return (uint32_t)(uintptr_t)(lds_void_t *)p;
}
__device__ __forceinline__ int32_t lds_read_i32(const int32_t *p) {
  int32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_off(p)) : "memory");
  return v;
}
__device__ __forceinline__ void lds_write_i32(int32_t *p, int32_t v) {
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)"
               :: "v"(lds_off(p)), "v"(v) : "memory");
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

constexpr uint32_t kLdsSpin = 1u << 20;   // polls before an LDS wait gives up

// the wavefront waits until the LDS word at p is at least v; false if it
// gave up after `spin` polls
__device__ __forceinline__ bool lds_wait_ge(const int32_t *p, int32_t v,
                                            uint32_t spin = kLdsSpin) {
  for (uint32_t n = 0; n < spin; ++n) {
    if (lds_read_i32(p) >= v) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// A barrier of wavefronts w0 .. w0+NW-1 only, in LDS: each posts its phase
// and polls the others', so wavefronts outside the group -- stalled behind
// their own weight loads -- are never waited for.  ok turns false if a poll
// gave up.  kSleep: back off between polls (for groups that wait long).
template <int NW, bool kSleep = true>
struct GroupSync {
  int32_t *flags;   // NW LDS words, zero before the first phase
  int w0;
  int phase;
  bool ok;
  __device__ void operator()() {
    const int lane = threadIdx.x & 63, wave = (threadIdx.x >> 6) - w0;
    ++phase;
    wait_lds();
    if (lane == 0) lds_write_i32(flags + wave, phase);
    bool done = false;
    for (uint32_t n = 0; n < kLdsSpin && !done; ++n) {
      done = __all(lds_read_i32(flags + lane % NW) >= phase);
      if (!done && kSleep) __builtin_amdgcn_s_sleep(1);
    }
    ok = ok && done;
  }
};

// One scale block (8 groups, fewer in the last block) of one tile, as held
// by one lane: its 16-byte scale row and 8 weight pieces of 32 weights.
struct BlockRegs {
  uint4 sc;
  uint4 w[kGroupsPerBlock];
};

__device__ __forceinline__ void load_block(BlockRegs &R, const uint8_t *bb, int ng,
                                           int lane) {
  R.sc = ldg16(bb + (lane >> 2) * 16);
  if (ng == kGroupsPerBlock) {
#pragma unroll
    for (int i = 0; i < kGroupsPerBlock; ++i)
      R.w[i] = ldg16(bb + kScaleChunk + i * kGroupChunk + lane * 16);
  } else {
#pragma unroll
    for (int i = 0; i < kGroupsPerBlock; ++i)
      if (i < ng) R.w[i] = ldg16(bb + kScaleChunk + i * kGroupChunk + lane * 16);
  }
}

template <int NG>
__device__ __forceinline__ int64_t dot_groups(const BlockRegs &R, int ng, int g0, int q,
                                              const int8_t *xs, const int32_t *xlo,
                                              int64_t p) {
#pragma unroll
  for (int i = 0; i < kGroupsPerBlock; ++i) {
    if (i < NG && (NG == kGroupsPerBlock || i < ng)) {
      const int g = g0 + i;
      const int s16 = dot_group(R.w[i], xs + kGroup * g + 32 * q, xlo[g * 4 + q]);
      p += (int64_t)(int32_t)scale_of(R.sc, i) * (int64_t)s16;
    }
    // a full block is scheduled as two halves: the x reads of four groups
    // are in flight together, and at most four groups' x are held at once
    if (NG == kGroupsPerBlock && i == kGroupsPerBlock / 2 - 1)
      __builtin_amdgcn_sched_barrier(0);
  }
  return p;
}

// A full block (8 groups; every block of K % 1024 == 0) takes a branch-free
// path, so the LDS reads of x for all its groups can be in flight together
// instead of one group's latency at a time.
__device__ __forceinline__ int64_t dot_block(const BlockRegs &R, int ng, int g0, int q,
                                             const int8_t *xs, const int32_t *xlo,
                                             int64_t p) {
  if (ng == kGroupsPerBlock) return dot_groups<kGroupsPerBlock>(R, ng, g0, q, xs, xlo, p);
  return dot_groups<kGroupsPerBlock - 1>(R, ng, g0, q, xs, xlo, p);
}

}  // namespace w4a8
