// Persistent decode-step kernel (W4A8_PLAN_PERSISTENT) for gfx950.
//
// One cooperative launch runs every site of a plan in order, one workgroup
// per CU: 8 weight wavefronts and 1 control wavefront.
//
//  * Weight wavefronts stream the weights and do the dot products.  The
//    weight blocks this CU owns over the whole plan form one fixed sequence
//    (its tiles of site 0, then of site 1, ...; 8448-byte scale blocks
//    within a tile), dealt round-robin to the 8 wavefronts.  Each wavefront
//    holds its next two blocks in two register sets, A and B, and refills a
//    set as soon as it has consumed it -- also when the next block belongs
//    to a later site, since weights never depend on an activation.  So the
//    next site's blocks stream while the workgroup waits for the rest of the
//    GPU and computes the next prologue.
//  * A weight wavefront makes no global access but its weight loads, and
//    every refill is the same 9 buffer loads (out of range, so without a
//    memory access, past the end of the sequence).  The compiler's count of
//    a wavefront's outstanding loads is therefore exact on every path, and
//    the wait for one register set never waits for the other.  Outputs,
//    error bits and the exported prologue vectors go through LDS.
//  * A tile's 16 rows are complete when every wavefront holding one of its
//    blocks has added its partial sums into an LDS slot; the wavefront that
//    completes the count rounds, checks and applies the epilogue, then
//    stages the outputs.  No workgroup barrier per tile.
//  * The control wavefront does every other global access: it stores the
//    staged outputs, signals this workgroup's completion of a site, waits for
//    all workgroups (one flag per workgroup), and copies the next site's
//    activation vector (and RMSNorm weights) into LDS.
//
// The LDS flags and the workgroup barriers are inline assembly: the
// compiler's own forms make a wavefront wait for all of its outstanding
// loads (vmcnt(0)), which would drain the register pipeline.  The data
// crossing a site boundary (outputs, activation vectors, flags) moves with
// agent-coherent accesses (sc1), so no cache-wide writeback or invalidation
// is needed.  Every result is bit-exact with the reference's integer law
// (ref/w4a8_ref.py:254-289 and the epilogues of gen_layer_script.py:1397-1433,
// seq_model.py:1027-1050).
#include "w4a8_device.h"

namespace w4a8 {

namespace {

constexpr int kCW = 8;                      // weight wavefronts
constexpr int kCtrl = kCW;                  // index of the control wavefront
constexpr int kThreads = (kCW + 1) * 64;    // 576
constexpr int kWThreads = kCW * 64;         // 512 threads run the prologue
constexpr int kPiece = kWThreads * 8;       // 4096 elements per prologue piece
constexpr int kXPieces = (kKMax + kPiece - 1) / kPiece;   // 3
constexpr int kXBytes = 2 * kKMax;          // x16 (24 KiB) / x8 + corrections
constexpr int kXloOff = kKMax;              // int32 corrections after x8
constexpr int kNormOff = 16384;             // RMSNorm weights (K <= 4096)
constexpr int kTSlots = 8;                  // tiles being reduced at once
constexpr uint32_t kGridSpin = 1u << 18;    // polls before a grid wait gives up
constexpr int kBufDword3 = 0x00020000;      // raw buffer, 32-bit data format

static_assert(kPiece % 32 == 0, "a DPP quad of threads covers one (group, quarter)");
static_assert(kStreamNormKMax <= kPiece, "RMSNorm takes one piece per thread");
static_assert(kNormOff + 2 * kStreamNormKMax <= kXBytes, "norm weights fit");
static_assert(kXloOff + 4 * kKMax / 32 <= kNormOff, "corrections fit");

// The site table is read-only for the whole launch.  Read through the
// constant address space, every (uniform) field load is a scalar load, also
// after barriers, so weight wavefronts never issue a vector load of their
// own besides the weight loads.
typedef const __attribute__((address_space(4))) GemvParams CSite;
typedef const __attribute__((address_space(4))) GemvJob CJob;

struct __align__(16) Lds {
  int8_t x[2][kXBytes];             // activations of site s in x[s & 1]
  int16_t xn[kStreamNormKMax];      // the site's RMSNorm output (workgroup 0 exports it)
  int64_t tv[kTSlots][kTileRows];   // partial sums, then staged outputs
  int32_t tcnt[kTSlots];            // contributions added to the slot
  int32_t tgen[kTSlots];            // tile number the slot is open for
  int32_t tready[kTSlots];          // tile number + 1 once its outputs are staged
  int32_t abort;                    // set by the first LDS wait that gives up
  int32_t err;                      // error bits found by the weight wavefronts
  uint16_t rsqrt[512];
  uint16_t sig[264];
  int64_t part[2][kCW];             // prologue partial reductions
  uint64_t best;                    // argmax key of the head's rows seen here (0: none)
};

// ---------------------------------------------------------------------------
// copies into LDS (control wavefront) and LDS synchronisation
// ---------------------------------------------------------------------------
// lane l copies 16 bytes from src (its own address) to LDS lds_base + 16 * l;
// lds_base must be uniform
__device__ __forceinline__ void copy16_sc1(const void *src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1"
               :: "v"(src), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void copy16(const void *src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void lds_add_u64(int64_t *p, int64_t v) {
  asm volatile("ds_add_u64 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_max_u64(uint64_t *p, uint64_t v) {
  asm volatile("ds_max_u64 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_or_i32(int32_t *p, int32_t v) {
  asm volatile("ds_or_b32 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}
__device__ __forceinline__ int32_t lds_add_rtn_i32(int32_t *p, int32_t v) {
  int32_t old;
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(old) : "v"(lds_off(p)), "v"(v) : "memory");
  return old;
}
// workgroup barrier for LDS data (this wavefront's LDS writes are done)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// lane 0 polls an LDS word until it equals v (or, with kAtLeast, until it
// is at least v).  Bounded: the first wait that
// gives up sets bit 2 of the error word and the workgroup's abort word,
// after which no wait of the workgroup polls again, so a launch always
// drains quickly.
template <bool kAtLeast = false>
__device__ __forceinline__ void lds_wait_eq(Lds &L, const int32_t *p, int v, int lane) {
  if (lane == 0) {
    uint32_t n = 0;
    for (;;) {
      const int32_t cur = lds_read_i32(p);
      if ((kAtLeast ? cur >= v : cur == v) || lds_read_i32(&L.abort) != 0) break;
      __builtin_amdgcn_s_sleep(1);
      if (++n > kLdsSpin) {
        lds_write_i32(&L.abort, 1);
        lds_or_i32(&L.err, 4);
        break;
      }
    }
  }
  wait_lds();
}

template <typename T>
__device__ __forceinline__ void store_coherent(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------- geometry
// This CU's share of a site: tiles first, first + G, ... (< total_tiles).
struct Cursor {
  int s;      // site; nsites once the sequence is exhausted
  int j;      // block index among the site's blocks on this CU
  int kt0;    // CU-local number of the site's first tile
  int nb;     // blocks of the site on this CU
  int ntl;    // tiles of the site on this CU
  int nblk;   // scale blocks per tile
  int first;  // first global tile of the site on this CU
};

__device__ __forceinline__ void cur_load_site(CSite *sites, int r, int G, Cursor &c) {
  CSite &P = sites[c.s];
  c.first = (r + P.tile_rot) % G;
  c.ntl = c.first < P.total_tiles ? (P.total_tiles - 1 - c.first) / G + 1 : 0;
  c.nblk = P.nblk;
  c.nb = c.ntl * c.nblk;
}

// move forward until block j lies in site s (or past the last site)
__device__ __forceinline__ void cur_settle(CSite *sites, int nsites, int r, int G, Cursor &c) {
  while (c.s < nsites && c.j >= c.nb) {
    c.j -= c.nb;
    c.kt0 += c.ntl;
    ++c.s;
    if (c.s < nsites) cur_load_site(sites, r, G, c);
  }
}

__device__ __forceinline__ void cur_init(CSite *sites, int nsites, int r, int G, int j0,
                                         Cursor &c) {
  c.s = 0;
  c.j = j0;
  c.kt0 = 0;
  c.nb = c.ntl = c.nblk = c.first = 0;
  if (nsites > 0) cur_load_site(sites, r, G, c);
  cur_settle(sites, nsites, r, G, c);
}

__device__ __forceinline__ void cur_next(CSite *sites, int nsites, int r, int G, Cursor &c) {
  c.j += kCW;
  cur_settle(sites, nsites, r, G, c);
}

// Put block c in flight into R: always the same 1 + kGroupsPerBlock buffer
// loads.  The buffer's range ends with the block's data, so for an item past
// the end of the sequence (range 0), and for the missing groups of a short
// block, the loads are out of range: they return zero without a memory
// access, and keep the count of outstanding loads the same on every path.
__device__ __forceinline__ void issue_block(BlockRegs &R, CSite *sites, int nsites, int G,
                                            const Cursor &c, int lane) {
  const uint8_t *bb = (const uint8_t *)sites[0].tables;   // any mapped address: range 0
  int len = 0;
  if (c.s < nsites) {
    CSite &P = sites[c.s];
    const int i = c.j / c.nblk, b = c.j - i * c.nblk;
    const int t = c.first + i * G;
    CJob &J = P.job[job_of(P, t)];
    bb = J.w + (int64_t)(t - J.tile0) * P.tile_bytes + (int64_t)b * kBlockBytes;
    len = kScaleChunk + groups_in(P.NG, b) * kGroupChunk;
  }
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void *)bb, (short)0, len, kBufDword3);
  const u32x4_t sc = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane >> 2) * 16, 0, kAuxNt);
  R.sc = make_uint4(sc.x, sc.y, sc.z, sc.w);
#pragma unroll
  for (int i = 0; i < kGroupsPerBlock; ++i) {
    const u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(
        rs, kScaleChunk + i * kGroupChunk + lane * 16, 0, kAuxNt);
    R.w[i] = make_uint4(w.x, w.y, w.z, w.w);
  }
}

// ------------------------------------------------------------- prologue
// The site's activation vector is in LDS buffer xb (int16 x at xb[0, 2K),
// int8 x at xb[0, K) for PRO_X8; RMSNorm weights at xb[kNormOff, +2K)).
// Leaves x8 at xb[0, K) and the offset corrections at xb[kXloOff] (and, in
// workgroup 0 when the site exports it, the RMSNorm output at L.xn); returns
// e_x.  All 9 wavefronts call it (the same barriers); the control wavefront
// computes nothing.
__device__ int stream_prologue(CSite &P, Lds &L, int8_t *xb, int tid, bool ctrl) {
  const int K = P.K;
  const int lane = tid & 63, wave = tid >> 6;
  int32_t *xlo = (int32_t *)(xb + kXloOff);
  if (P.pro == PRO_X8) {
    if (!ctrl) {
      for (int c = tid; c < P.NG * 4; c += kWThreads) {
        const int *xw = (const int *)(xb + 32 * c);
        int s = 0;
        s = __builtin_amdgcn_sdot4(xw[0], 0x01010101, s, false);
        s = __builtin_amdgcn_sdot4(xw[2], 0x01010101, s, false);
        s = __builtin_amdgcn_sdot4(xw[4], 0x01010101, s, false);
        s = __builtin_amdgcn_sdot4(xw[6], 0x01010101, s, false);
        xlo[c] = -8 * s;
      }
    }
    lds_barrier();
    return P.e_x_given;
  }
  const int np = (K + kPiece - 1) / kPiece;
  int4 pc[kXPieces];
#pragma unroll
  for (int c = 0; c < kXPieces; ++c) {
    const int base = c * kPiece + tid * 8;
    pc[c] = make_int4(0, 0, 0, 0);
    if (!ctrl && c < np && base < K) pc[c] = *(const int4 *)(xb + 2 * base);
  }
  if (P.pro == PRO_RMSNORM_DYNQ8) {
    // layer_fixed.py:1262-1278 in sign-magnitude form (rshift_round rounds
    // the magnitude); K <= kStreamNormKMax, so one piece per thread
    const int base = tid * 8;
    int4 wv = make_int4(0, 0, 0, 0);
    if (!ctrl && base < K) wv = *(const int4 *)(xb + kNormOff + 2 * base);
    uint64_t ss = 0;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const int32_t a = piece_get(pc[0], j), b = piece_get(pc[0], j + 1);
      ss += (uint64_t)((uint32_t)(a * a) + (uint32_t)(b * b));
    }
    ss = wave_sum_u64(ss);
    if (!ctrl && lane == 0) L.part[0][wave] = (int64_t)ss;
    lds_barrier();
    ss = 0;
#pragma unroll
    for (int w = 0; w < kCW; ++w) ss += (uint64_t)L.part[0][w];
    if (ss == 0) ss = 1;
    int64_t r;
    int e;
    rsqrt_q(ss, 2 * P.in_f + (31 - __clz(K)), L.rsqrt, &r, &e);
    const int s1 = 30 - e;
    const int32_t one = P.one_plus ? (1 << 14) : 0;
    const int rs = s1 < 0 ? 0 : (s1 > 63 ? 63 : s1);
    const int ls = s1 < 0 ? (-s1 > 63 ? 63 : -s1) : 0;
    const uint64_t half1 = rs > 0 ? ((uint64_t)1 << (rs - 1)) : 0;
    const bool right = s1 >= 0;
    // r < 2^31 (a Q30 reciprocal square root), |x| <= 2^15; for in_f within
    // 0..40 (checked on the host) the left shift is at most 17, so |x| * r
    // shifted stays below 2^63
    const uint32_t r32 = (uint32_t)r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int32_t xv = piece_get(pc[0], j);
      const int32_t sc = (int32_t)piece_get(wv, j) + one;
      const uint64_t mag = (uint64_t)(uint32_t)abs(xv) * (uint64_t)r32;
      uint64_t ym = right ? ((mag + half1) >> rs) : (mag << ls);
      // y is clipped to [-2^32, 2^32 - 1]; a magnitude of 2^32 or more
      // saturates the int16 result below for any nonzero scale, exactly as
      // 2^32 - 1 does, so the product can be formed in 32 x 32 bits
      ym = ym < 0xFFFFFFFFull ? ym : 0xFFFFFFFFull;
      const uint64_t q = ((uint64_t)(uint32_t)ym * (uint64_t)(uint32_t)abs(sc) + 8192u) >> 14;
      const bool neg = (xv < 0) != (sc < 0);
      const int32_t q32 = q > 65535u ? 65535 : (int32_t)q;
      const int32_t qm = min(q32, 32767 + (int32_t)neg);
      piece_set(pc[0], j, (int16_t)(neg ? -qm : qm));
    }
    if (!ctrl && blockIdx.x == 0 && P.xn_out && base < K) *(int4 *)(L.xn + base) = pc[0];
  }
  int32_t mx = 0;
#pragma unroll
  for (int c = 0; c < kXPieces; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = max(mx, abs((int32_t)piece_get(pc[c], j)));
  mx = wave_max_i32(mx);
  if (!ctrl && lane == 0) L.part[1][wave] = mx;
  lds_barrier();
  mx = 0;
#pragma unroll
  for (int w = 0; w < kCW; ++w) mx = max(mx, (int32_t)L.part[1][w]);
  // fixedpoint.py:24-33: the least e with rshift_round(max, e) <= 127 is
  // bitlen(max) - 7, or one more when rounding carries past 127
  int e = mx > 127 ? 25 - __clz(mx) : 0;
  if (e > 0 && ((mx + (1 << (e - 1))) >> e) > 127) ++e;
  const int32_t half = (1 << e) >> 1;
  if (!ctrl) {
#pragma unroll
    for (int c = 0; c < kXPieces; ++c) {
      const int base = c * kPiece + tid * 8;
      if (c < np) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int32_t v = piece_get(pc[c], j);
          const int32_t qm = min((abs(v) + half) >> e, 127);
          const uint32_t b8 = (uint32_t)(uint8_t)(int8_t)(v < 0 ? -qm : qm);
          if (j < 4) lo |= b8 << (8 * j);
          else       hi |= b8 << (8 * (j - 4));
        }
        // -8 * sum of the x8 met by the offset-form low nibbles of one
        // (group, quarter): 32 consecutive k = the 4 threads of a DPP quad
        int t4 = __builtin_amdgcn_sdot4((int)lo, 0x01010101, 0, false);
        t4 += __builtin_amdgcn_update_dpp(0, t4, 0xB1, 0xF, 0xF, false);
        t4 += __builtin_amdgcn_update_dpp(0, t4, 0x4E, 0xF, 0xF, false);
        if (base < K) {
          *(uint2 *)(xb + base) = make_uint2(lo, hi);
          if ((tid & 3) == 0) xlo[base / 32] = -8 * t4;
        }
      }
    }
  }
  lds_barrier();
  return e;
}

// ------------------------------------------------------------- tiles
// Add this wavefront's share of tile kt; true if it completed the tile.
__device__ __forceinline__ bool tile_add(Lds &L, int kt, int64_t p, int contributors,
                                         int lane) {
  const int slot = kt & (kTSlots - 1);
  lds_wait_eq(L, &L.tgen[slot], kt, lane);
  // rows: lanes 4r..4r+3 hold the 4 k-quarters of row r
  p = (int64_t)((uint64_t)p + dpp_u64<0xB1, 0xF>((uint64_t)p));
  p = (int64_t)((uint64_t)p + dpp_u64<0x4E, 0xF>((uint64_t)p));
  if ((lane & 3) == 0) lds_add_u64(&L.tv[slot][lane >> 2], p);
  int old = 0;
  if (lane == 0) old = lds_add_rtn_i32(&L.tcnt[slot], 1);
  old = __builtin_amdgcn_readfirstlane(old);
  return old == contributors - 1;
}

// The completing wavefront: round, check and apply the epilogue to the 16
// rows of tile kt (tile tl of job J).  Argmax tiles fold their rows into the
// workgroup's key in LDS and free the slot; the others are staged for the
// control wavefront.
__device__ __forceinline__ void tile_epilogue(Lds &L, int kt, CJob &J, int tl, int e_x,
                                              int lane) {
  const int slot = kt & (kTSlots - 1);
  const bool argmax = J.epi == EPI_ARGMAX;
  if (lane < kTileRows) {
    const int64_t tot = L.tv[slot][lane];
    const int row = tl * kTileRows + lane;
    int64_t outv = 0;
    if (row < J.nrows) {
      const int64_t y = rshr64(tot >> 4, J.sh);   // tot is 16 * p exactly
      if (y > 2147483647LL || y < -2147483647LL) lds_or_i32(&L.err, 1);
      const int shift = J.p0 - e_x;
      switch (J.epi) {
        case EPI_Y32: outv = y; break;
        case EPI_MOVY_I16: outv = clamp64(movy_shift(y, shift), -32768, 32767); break;
        case EPI_MOVY_P32:
          outv = clamp64(movy_shift(y, shift), -2147483648LL, 2147483647LL);
          break;
        case EPI_SILU32: outv = silu32(y, shift, L.sig); break;
        case EPI_SHIFT_I64: outv = movy_shift(y, shift); break;
        default:   // EPI_ARGMAX: raw y32, seq_format.py:2225-2226
          lds_max_u64(&L.best, argmax_key((int32_t)y, (uint32_t)row));

      }
    }
    L.tv[slot][lane] = argmax ? 0 : outv;
  }
  if (lane == 0) {
    if (argmax) {
      lds_write_i32(&L.tcnt[slot], 0);
      lds_write_i32(&L.tgen[slot], kt + kTSlots);
    } else {
      lds_write_i32(&L.tready[slot], kt + 1);
    }
  }
  wait_lds();
}

// ------------------------------------------------------------- control
// start copying the site's activation vector (agent-coherent) and RMSNorm
// weights into LDS buffer xb; the caller waits (vmcnt) before the barrier
// that hands the buffer to the weight wavefronts
__device__ __forceinline__ void ctrl_issue_inputs(CSite &P, int8_t *xb, int lane) {
  const uint8_t *x = (const uint8_t *)P.x;
  const int nb = P.pro == PRO_X8 ? P.K : 2 * P.K;
  for (int off = 0; off < nb; off += 1024)
    if (off + 16 * lane < nb) copy16_sc1(x + off + 16 * lane, lds_off(xb + off));
  if (P.pro == PRO_RMSNORM_DYNQ8) {
    const uint8_t *w = (const uint8_t *)P.norm_w;
    for (int off = 0; off < 2 * P.K; off += 1024)
      if (off + 16 * lane < 2 * P.K) copy16(w + off + 16 * lane, lds_off(xb + kNormOff + off));
  }
}

// workgroup 0: the prologue's exported vectors (x8, the RMSNorm output, e_x)
__device__ void ctrl_export(CSite &P, Lds &L, const int8_t *xb, int e_x, int lane) {
  const int K = P.K;
  if (P.x8_out)
    for (int off = 16 * lane; off < K; off += 1024) {
      const int4 v = *(const int4 *)(xb + off);
      int32_t *o = (int32_t *)(P.x8_out + off);
      store_coherent(o, v.x);
      store_coherent(o + 1, v.y);
      store_coherent(o + 2, v.z);
      store_coherent(o + 3, v.w);
    }
  if (P.pro == PRO_RMSNORM_DYNQ8 && P.xn_out)
    for (int i = 8 * lane; i < K; i += 512) {
      const int4 v = *(const int4 *)(L.xn + i);
      int32_t *o = (int32_t *)(P.xn_out + i);
      store_coherent(o, v.x);
      store_coherent(o + 1, v.y);
      store_coherent(o + 2, v.z);
      store_coherent(o + 3, v.w);
    }
  if (P.e_x_out && lane == 0) store_coherent(P.e_x_out, (int32_t)e_x);
}

// Store the outputs of this CU's tiles of site P (tile numbers kt0, ...).
// Argmax tiles stage nothing: their slot is freed by the wavefront that
// completes them, which is waited for here too, so that no wavefront still
// reads this site's activations once this returns.
__device__ void ctrl_serve(CSite &P, Lds &L, int kt0, int r, int G, int lane) {
  const int first = (r + P.tile_rot) % G;
  for (int i = 0, t = first; t < P.total_tiles; ++i, t += G) {
    CJob &J = P.job[job_of(P, t)];
    const int kt = kt0 + i, slot = kt & (kTSlots - 1);
    if (J.epi == EPI_ARGMAX) {
      // later argmax tiles may have reused and freed the slot since
      lds_wait_eq<true>(L, &L.tgen[slot], kt + kTSlots, lane);
      continue;
    }
    lds_wait_eq(L, &L.tready[slot], kt + 1, lane);
    if (lane < kTileRows) {
      const int64_t v = L.tv[slot][lane];
      const int row = (t - J.tile0) * kTileRows + lane;
      if (row < J.nrows) {
        switch (J.epi) {
          case EPI_MOVY_I16:
          case EPI_SILU32: store_coherent((int16_t *)J.out + row, (int16_t)v); break;
          case EPI_SHIFT_I64: store_coherent((int64_t *)J.out + row, v); break;
          default: store_coherent((int32_t *)J.out + row, (int32_t)v); break;
        }
      }
      L.tv[slot][lane] = 0;
    }
    if (lane == 0) {
      lds_write_i32(&L.tcnt[slot], 0);
      lds_write_i32(&L.tgen[slot], kt + kTSlots);
    }
  }
}

// all G workgroups have stored flag value >= v (bounded; bit 1 of err)
__device__ void grid_wait(uint32_t *flags, int G, uint32_t v, int lane, int32_t *err) {
  uint32_t n = 0;
  for (;;) {
    bool ok = true;
    for (int i = lane; i < G; i += 64)
      ok = ok && __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= v;
    if (__all(ok)) break;
    __builtin_amdgcn_s_sleep(1);
    if (++n > kGridSpin) {
      if (lane == 0) atomicOr(err, 2);
      break;
    }
  }
}

__global__ __launch_bounds__(kThreads) void stream_kernel(StreamParams S,
                                                          const GemvParams *__restrict__ sites_arg) {
  CSite *sites = (CSite *)sites_arg;
  __shared__ Lds L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool ctrl = wave == kCtrl;
  const int G = gridDim.x, r = blockIdx.x;
  const int nsites = S.nsites;

  // tables and reduction slots
  const int32_t *tab = sites[0].tables;
  for (int i = tid; i < 512; i += kThreads) L.rsqrt[i] = (uint16_t)tab[kRsqrtOff + i];
  for (int i = tid; i < 257; i += kThreads) L.sig[i] = (uint16_t)tab[kSigmoidOff + i];
  for (int i = tid; i < kTSlots * kTileRows; i += kThreads) (&L.tv[0][0])[i] = 0;
  if (tid < kTSlots) {
    L.tcnt[tid] = 0;
    L.tgen[tid] = tid;
    L.tready[tid] = 0;
  }
  if (tid == 0) {
    L.abort = 0;
    L.err = 0;
    L.best = 0;
  }
  wait_vm_all();   // the table loads, before any weight load is counted

  if (ctrl) {
    // Site s's activations go to x[s & 1].  Unless site s+1 is fenced, its
    // activations are copied into the other buffer while site s computes
    // (every weight wavefront is past site s-1, the buffer's last user); a
    // fenced site first waits until every workgroup has stored its outputs
    // of all earlier sites (flag value s+1), then copies.
    int kt0 = 0;   // CU-local number of the site's first tile
    if (nsites > 0) ctrl_issue_inputs(sites[0], L.x[0], lane);
    wait_vm_all();
    for (int s = 0; s < nsites; ++s) {
      CSite &P = sites[s];
      int8_t *xb = L.x[s & 1];
      lds_barrier();   // site s's activation vector is in LDS
      if (S.trace && r == 0 && lane == 0) S.trace[s] = wall_clock64();
      const bool ahead = s + 1 < nsites && !sites[s + 1].fence;
      if (ahead) ctrl_issue_inputs(sites[s + 1], L.x[(s + 1) & 1], lane);
      const int e_x = stream_prologue(P, L, xb, tid, true);
      if (r == 0) ctrl_export(P, L, xb, e_x, lane);
      // the next site's activations have landed (this site's output stores,
      // issued below, are only waited for at a fence)
      wait_vm_all();
      ctrl_serve(P, L, kt0, r, G, lane);
      {
        const int first = (r + P.tile_rot) % G;
        kt0 += first < P.total_tiles ? (P.total_tiles - 1 - first) / G + 1 : 0;
      }
      if (s + 1 < nsites && !ahead) {
        wait_vm_all();   // outputs stored
        if (lane == 0) store_coherent(S.done + r, (uint32_t)(s + 1));
        grid_wait(S.done, G, (uint32_t)(s + 1), lane, S.err);
        ctrl_issue_inputs(sites[s + 1], L.x[(s + 1) & 1], lane);
        wait_vm_all();
      }
    }
  } else {
    // A holds item k of this wavefront's sequence, B item k + 1; cn is the
    // next item to put in flight
    Cursor ca, cb, cn;
    cur_init(sites, nsites, r, G, wave, ca);
    cb = ca;
    cur_next(sites, nsites, r, G, cb);
    cn = cb;
    cur_next(sites, nsites, r, G, cn);
    BlockRegs A, B;
    issue_block(A, sites, nsites, G, ca, lane);
    issue_block(B, sites, nsites, G, cb, lane);
    int s_cur = -1, e_x = 0, contributors = 0;
    int64_t p = 0;
    // join site s's barriers and compute its prologue; the lane-derived
    // addresses are recomputed from an opaque copy of the thread index, so
    // the compiler does not keep them all live across the whole plan
    auto enter = [&](int s) {
      int tid_s = tid;
      asm volatile("" : "+v"(tid_s));
      lds_barrier();   // site s's activation vector is in LDS
      e_x = stream_prologue(sites[s], L, L.x[s & 1], tid_s, false);
      contributors = min(sites[s].nblk, kCW);
    };
    // consume the block in R (item c; this wavefront's next item is nx),
    // refill R with the item two ahead, and add into the tile after this
    // wavefront's last block of it
    auto step = [&](BlockRegs &R, Cursor &c, const Cursor &nx) {
      while (s_cur < c.s) enter(++s_cur);
      int tid_s = tid;
      asm volatile("" : "+v"(tid_s));
      const int lane_s = tid_s & 63;
      CSite &P = sites[c.s];
      const int i = c.j / c.nblk, b = c.j - i * c.nblk;
      const int8_t *xb = L.x[c.s & 1];
      p = dot_block(R, groups_in(P.NG, b), b * kGroupsPerBlock, lane_s & 3, xb,
                    (const int32_t *)(xb + kXloOff), p);
      const bool last = !(nx.s == c.s && nx.j / nx.nblk == i);
      const Cursor done = c;
      c = cn;
      cur_next(sites, nsites, r, G, cn);
      issue_block(R, sites, nsites, G, c, lane_s);
      if (last) {
        const int kt = done.kt0 + i;
        if (tile_add(L, kt, p, contributors, lane_s)) {
          const int t = done.first + i * G;
          CJob &J = P.job[job_of(P, t)];
          tile_epilogue(L, kt, J, t - J.tile0, e_x, lane_s);
        }
        p = 0;
      }
    };
    for (;;) {
      if (ca.s >= nsites) break;
      step(A, ca, cb);
      if (cb.s >= nsites) break;
      step(B, cb, ca);
    }
    // sites after this wavefront's last block: it still joins their barriers
    while (s_cur < nsites - 1) enter(++s_cur);
  }

  int tid_e = tid;
  asm volatile("" : "+v"(tid_e));
  const int lane_e = tid_e & 63;
  lds_barrier();
  if (ctrl && lane_e == 0) {
    const int32_t e = lds_read_i32(&L.err);
    if (e) atomicOr(S.err, e);
    if (S.head_site >= 0) S.partials[r] = L.best;
  }
  if (S.trace && r == 0 && ctrl && lane_e == 0) S.trace[nsites] = wall_clock64();
}

}  // namespace

hipError_t launch_stream(const StreamParams &sp, int grid, hipStream_t s) {
  const GemvParams *sites = sp.sites;
  void *args[] = {(void *)&sp, (void *)&sites};
  return hipLaunchCooperativeKernel((const void *)stream_kernel, dim3(grid), dim3(kThreads),
                                    args, 0, s);
}

int stream_max_blocks_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, stream_kernel, kThreads, 0) !=
          hipSuccess || n < 1)
    n = 1;
  return n > 1 ? 1 : n;
}

size_t stream_counter_words(int grid) { return (size_t)(grid + 63) / 64 * 64; }

}  // namespace w4a8
