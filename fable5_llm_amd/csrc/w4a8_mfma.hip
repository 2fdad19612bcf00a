// Batched W4A8 (several tokens): int8 MFMA on gfx950 with the per-group
// scale applied after accumulation.  Per token the result is bit-identical
// to ref/w4a8_ref.py:254-289 matvec_y32: every group sum is exact in int32
// (|16 * sum w*x| <= 2^21) and the scale products are summed exactly (in
// int64 or, below 2^53, in double precision).
//
// v_mfma_i32_16x16x64_i8: A = 16 weight rows x 64 k, B = 64 k x 16 tokens,
// D = 16 x 16 int32.  Lane l feeds row/token (l % 16) and k-quarter l / 16
// of A and B alike, so A and B share one lane->k mapping and the dot product
// does not depend on the order in which the hardware walks k.  D element
// (4 * (l / 16) + r, l % 16) lands in lane l, register r.
//
// One workgroup per CU, 12 wavefronts:
//
//  * 8 group wavefronts.  A tile's scale block b covers groups 8b..8b+7;
//    wavefront w takes group 8b + w of every block, so the 8 read one
//    block's 8 KiB of weights together.  Each keeps its next kMD 16-byte
//    weight pieces in flight (uniform buffer loads: the compiler's count of
//    its outstanding loads is exact, and a wait is for the oldest piece
//    only).
//  * up to 3 loader wavefronts copy, with LDS DMA, each block's activations
//    (B tokens x 1 KiB) and the scale rows of the round's tiles into a ring
//    of LDS slots, ahead of the group wavefronts, and flag each slot once its
//    copies have landed.
//  * 1 store wavefront: at the end of a round the 8 group wavefronts add
//    their sums into an LDS table (two tables, alternating by round);
//    the store wavefront rounds, checks and stores the round's y32 and frees
//    the table.  Group wavefronts thus issue no stores, which would make the
//    compiler's count of their outstanding loads unknown.
//
// A workgroup works through its tiles in rounds of up to TM tiles (TM * CT
// <= 4, CT = column tiles of 16 tokens), block-major within a round, so that
// each block's activations serve every tile of the round.  One launch may
// carry several matrices (jobs, same tokens, each its own activations): a
// workgroup's rounds run through its tiles of job 0, then job 1, ..., and
// the ring, the loaders and the weight pieces in flight run on across the
// job boundaries, so the weight stream does not drain between matrices.  Every wait between wavefronts is bounded: a wait that gives
// up sets bit 2 of the error word and an abort word, after which no wait of
// the workgroup polls again, so a launch always drains.
#include <type_traits>
#include <vector>

#include "w4a8_device.h"

namespace w4a8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMW = 8;                     // group wavefronts 0..7
constexpr int kML = 3;                     // loader wavefronts 8..10 (at most)
constexpr int kMStore = kMW + kML;         // the store wavefront, 11
constexpr int kMThreads = (kMW + kML + 1) * 64;
constexpr int kXRow = 1024 + 16;           // LDS bytes per token of a block's activations
constexpr int kMBufDword3 = 0x00020000;    // raw buffer, 32-bit data format
constexpr int kMAuxNt = 2;                 // buffer-load cache policy: non-temporal
constexpr int kRingMax = 8;
constexpr int kLdsBytes = 160 * 1024;

static_assert(kXRow % 16 == 0, "token rows stay 16-byte aligned");

struct MmJob {
  const uint8_t *W;     // tile layout
  const int8_t *x8;     // [B][K]
  int32_t *y32;         // [B][nrows]
  int64_t tile_bytes;
  int32_t nrows, ntiles, NG, nblk, sh, K;
  int32_t tm;           // tiles per round
  int32_t ns;           // K slices (1: none), see the split below
  int64_t *part;        // split: [ns][B][nrows] each slice's sums (16 p)
};

// A split job (ns > 1; a matrix with at most one tile per workgroup) cuts
// K into ns slices of nblk / ns blocks.  Workgroup r takes slice r % ns of
// row tiles r / ns, r / ns + G / ns, ...: its rounds' tiles share one copy
// of the slice's activations, and a workgroup reads only its slice, the
// same one on every workgroup of its XCD (r % 8, with ns dividing 8).  Each
// slice stores its sums to part; matmul_finish_kernel adds the ns slices,
// rounds, checks and stores y32 after the launch.
struct MmSlice {
  int tr, tg, kb0, nbs;   // first row tile, row-tile stride, first block, blocks
  // ns is 1, 2 or 4 (the host's choice), so the divisions are shifts
  __device__ MmSlice(const MmJob &J, int r, int G) {
    const int l = __builtin_ctz((unsigned)J.ns);
    tr = r >> l;
    tg = G >> l;
    nbs = J.nblk >> l;
    kb0 = (r & (J.ns - 1)) * nbs;
  }
};

struct MmParams {
  MmJob job[kMmJobs];   // the jobs, when they travel in the parameters ...
  const MmJob *tab;     // ... or a device table of njobs (a matmul plan)
  int32_t njobs;
  int32_t B, CT;
  int32_t R;            // LDS slots
  int32_t nl;           // loader wavefronts in use
  int32_t slot_bytes;   // 16 * CT token rows of kXRow, then tm scale rows of 256 B
  int32_t *err;
};

// LDS: flags, then the reduction tables, then the ring of slots
struct MmFlags {
  int32_t ready[kRingMax];   // step whose copies have landed in the slot (-1: none)
  int32_t done[kMW];         // last step each group wavefront has finished (-1: none)
  int32_t tgen[2];           // round allowed to add into each table next
  int32_t tcnt[2];           // group wavefronts that have added this round
  int32_t abort;
  int32_t err;
  int32_t pad[2];
  // this workgroup's schedule: job j has nmine[j] of its tiles, global
  // rounds rbase[j] .. rbase[j + 1] - 1 and steps sbase[j] .. sbase[j + 1] - 1
  int32_t nmine[kMmPlanJobs];
  int32_t rbase[kMmPlanJobs + 1];
  int32_t sbase[kMmPlanJobs + 1];
};
static_assert(kMmPlanJobs <= 128, "the schedule scan takes two jobs a lane");
constexpr int kFlagBytes = (int)((sizeof(MmFlags) + 255) / 256 * 256);

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

__device__ __forceinline__ void mm_wait_vm_all() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ void mm_lds_add(double *p, double v) {
  asm volatile("ds_add_f64 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}
__device__ __forceinline__ void mm_lds_add(int64_t *p, int64_t v) {
  asm volatile("ds_add_u64 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}

// The sums of scale x group products of a kernel instance: exact either
// way (every product < 2^16 * 2^21, every partial sum < 96 groups * 2^37 <
// 2^44: integers below 2^53), in double precision (full-rate FMAs) where two
// or more column tiles give each scale several products, else in int64
// (quarter-rate multiply-adds, but no conversions)
template <int CTX>
using MmAcc = typename std::conditional<(CTX >= 2), double, int64_t>::type;
template <int CTX>
__device__ __forceinline__ MmAcc<CTX> mm_scale(int32_t m) { return (MmAcc<CTX>)m; }
__device__ __forceinline__ double mm_fma(double m, int32_t a, double p) {
  return __builtin_fma(m, (double)a, p);
}
__device__ __forceinline__ int64_t mm_fma(int64_t m, int32_t a, int64_t p) {
  return p + m * (int64_t)a;
}
__device__ __forceinline__ int32_t mm_lds_add_rtn(int32_t *p, int32_t v) {
  int32_t old;
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(old) : "v"(lds_off(p)), "v"(v) : "memory");
  return old;
}
// an LDS add that does not wait for itself (nor for earlier LDS work)
__device__ __forceinline__ void mm_lds_add_post(int32_t *p, int32_t v) {
  asm volatile("ds_add_u32 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}
// an LDS write that does not wait for itself (nor for earlier LDS work: a
// wavefront's LDS instructions execute in order)
__device__ __forceinline__ void mm_lds_post(int32_t *p, int32_t v) {
  asm volatile("ds_write_b32 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}
__device__ __forceinline__ void mm_lds_or(int32_t *p, int32_t v) {
  asm volatile("ds_or_b32 %0, %1" :: "v"(lds_off(p)), "v"(v) : "memory");
}
// lane l copies 16 (or 4) bytes from its own address to LDS lds_base + 16 l
// (4 l); lds_base must be uniform
__device__ __forceinline__ void dma16(const void *src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void *src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
               :: "v"(src), "s"(lds_base) : "memory", "m0");
}

// Bounded LDS wait of one wavefront: until every lane's predicate holds,
// the workgroup aborts, or kLdsSpin polls (then bit 2 of err and abort).
template <typename Pred>
__device__ __forceinline__ bool mm_wait(MmFlags &F, Pred pred) {
  for (uint32_t n = 0;; ++n) {
    if (__all(pred())) return true;
    if (lds_read_i32(&F.abort) != 0) return false;
    if (n > kLdsSpin) {
      if ((threadIdx.x & 63) == 0) {
        lds_write_i32(&F.abort, 1);
        mm_lds_or(&F.err, 4);
      }
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// The same wait for a group wavefront, as a loop of plain exits (the form
// in which the compiler keeps its count of outstanding weight loads across
// it): until the LDS word at p is at least v (kAtLeast) or equal to v.
template <bool kAtLeast>
__device__ __forceinline__ void mm_wait_word(MmFlags &F, const int32_t *p, int v, int lane) {
  for (uint32_t n = 0;; ++n) {
    const int32_t cur = lds_read_i32(p);
    if (__all(kAtLeast ? cur >= v : cur == v)) break;
    if (lds_read_i32(&F.abort) != 0) break;
    if (n > kLdsSpin) {
      if (lane == 0) {
        lds_write_i32(&F.abort, 1);
        mm_lds_or(&F.err, 4);
      }
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// A workgroup's tiles of a job are r, r + G, ...; the job's round rho takes
// tiles rho*tm .. rho*tm + nt - 1 of them, and the job's step
// rho * nblk + kb covers block kb of every tile of round rho.
__device__ __forceinline__ int round_tiles(const MmJob &J, int nmine, int rho) {
  return min(J.tm, nmine - rho * J.tm);
}

// Position in this workgroup's schedule: job j, its round rho and block kb;
// RHO counts rounds over all jobs.  Jobs with no tile on this workgroup are
// skipped.  The fields of job j that a step needs stay in registers, so the
// job table and the schedule in LDS are read only when the job changes (a
// read on every step puts its latency on every step).
struct MmCur {
  int j, rho, kb, RHO;     // kb: block of the slice (kb0 + kb of the matrix)
  int rend;                // first round past job j
  int nblk, tm, nmine, nt, NG, K;
  int tr, tg, kb0;         // the workgroup's slice (MmSlice; nblk = its blocks)
  const uint8_t *W;
  const int8_t *x8;
  int64_t tile_bytes;
  template <class JobF>
  __device__ void load(const MmFlags &F, int njobs, JobF &JOB) {
    if (j >= njobs) return;
    const MmJob &J = JOB(j);
    const MmSlice S(J, (int)blockIdx.x, (int)gridDim.x);
    tr = S.tr;
    tg = S.tg;
    kb0 = S.kb0;
    nblk = S.nbs;
    tm = J.tm;
    NG = J.NG;
    K = J.K;
    W = J.W;
    x8 = J.x8;
    tile_bytes = J.tile_bytes;
    nmine = __builtin_amdgcn_readfirstlane(F.nmine[j]);
    rend = __builtin_amdgcn_readfirstlane(F.rbase[j + 1]);
    nt = min(tm, nmine - rho * tm);
  }
  template <class JobF>
  __device__ void start(const MmFlags &F, int njobs, JobF &JOB) {
    j = 0;
    rho = kb = RHO = 0;
    nt = 0;
    W = nullptr;
    while (j < njobs && F.rbase[j + 1] == 0) ++j;
    load(F, njobs, JOB);
  }
  template <class JobF>
  __device__ void next(const MmFlags &F, int njobs, JobF &JOB) {
    if (++kb < nblk) return;
    kb = 0;
    ++rho;
    ++RHO;
    if (RHO < rend) {
      nt = min(tm, nmine - rho * tm);
      return;
    }
    rho = 0;
    while (j < njobs && RHO == F.rbase[j + 1]) ++j;
    load(F, njobs, JOB);
  }
};

// Put group 8 kb + w of tile j of the cursor's round in flight: a buffer
// load whose range is empty (no memory access, zeros) when there is no such
// tile or group, so every step issues the same loads.
__device__ __forceinline__ uint4 mm_issue(const MmCur &C, int r, int G, int w, int lane, int j,
                                          bool real) {
  const uint8_t *base = C.W;
  int len = 0;
  const int kb = C.kb0 + C.kb;
  if (real && 8 * kb + w < C.NG) {
    const int64_t t = (int64_t)C.tr + (int64_t)C.tg * (C.rho * C.tm + j);
    base = C.W + t * C.tile_bytes + (int64_t)kb * kBlockBytes + kScaleChunk +
           (int64_t)w * kGroupChunk;
    len = kGroupChunk;
  }
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, len, kMBufDword3);
  // lane (c = l % 16, q = l / 16) takes row c's quarter q: bytes (4c + q) * 16
  const int piece = ((lane & 15) * 4 + (lane >> 4)) * 16;
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, piece, 0, kMAuxNt);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// steps in flight per group wavefront: TMX pieces each (one tile a round,
// as for a matrix with no more tiles than workgroups, goes 8 steps deep)
template <int TMX, int CTX>
constexpr int mm_depth() { return TMX >= 3 ? 4 : 8; }

template <int TMX, int CTX, bool kTab>
__global__ __launch_bounds__(kMThreads) void matmul_kernel(MmParams P) {
  extern __shared__ __align__(16) uint8_t smem[];
  // job j (j uniform): from the parameters, or from the plan's device table
  // read as constant memory, so that its fields come in by scalar loads and
  // no wait for them counts the weight pieces in flight
  typedef const __attribute__((address_space(4))) MmJob CJob;
  auto JOB = [&](int j) -> const MmJob & {
    const int ju = __builtin_amdgcn_readfirstlane(j);
    if constexpr (kTab)
      return *(const MmJob *)((CJob *)P.tab + ju);
    else
      return P.job[ju];
  };
  MmFlags &F = *(MmFlags *)smem;
  typedef MmAcc<CTX> Acc;
  Acc *tables = (Acc *)(smem + kFlagBytes);   // [2][TMX][CTX][4][64]
  uint8_t *ring = smem + kFlagBytes + 2 * TMX * CTX * 4 * 64 * 8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, r = blockIdx.x;

  if (tid < kRingMax) F.ready[tid] = -1;
  if (tid < kMW) F.done[tid] = -1;
  if (tid < 2) {
    F.tgen[tid] = tid;
    F.tcnt[tid] = 0;
  }
  if (tid == 0) {
    F.abort = 0;
    F.err = 0;
  }
  // thread j: job j's tiles, rounds and steps on this workgroup ...
  if (tid < P.njobs) {
    const MmJob &J = kTab ? P.tab[tid] : P.job[tid];
    const MmSlice S(J, r, G);
    const int nm = S.tr < J.ntiles ? (J.ntiles - 1 - S.tr) / S.tg + 1 : 0;
    const int nr = (nm + J.tm - 1) / J.tm;
    F.nmine[tid] = nm;
    F.rbase[tid + 1] = nr;
    F.sbase[tid + 1] = nr * S.nbs;
  }
  for (int i = tid; i < 2 * TMX * CTX * 4 * 64; i += kMThreads) tables[i] = 0;
  __syncthreads();
  // ... and wavefront 0's prefix sums of them (lane l: jobs 2l, 2l + 1)
  if (wave == 0) {
    const int j0 = 2 * lane, j1 = 2 * lane + 1;
    const int a0 = j0 < P.njobs ? F.rbase[j0 + 1] : 0, b0 = j0 < P.njobs ? F.sbase[j0 + 1] : 0;
    const int a1 = j1 < P.njobs ? F.rbase[j1 + 1] : 0, b1 = j1 < P.njobs ? F.sbase[j1 + 1] : 0;
    int sa = a0 + a1, sb = b0 + b1;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int ta = __shfl_up(sa, o), tb = __shfl_up(sb, o);
      if (lane >= o) {
        sa += ta;
        sb += tb;
      }
    }
    const int ea = sa - a0 - a1, eb = sb - b0 - b1;   // before job j0
    if (j0 < P.njobs) {
      F.rbase[j0 + 1] = ea + a0;
      F.sbase[j0 + 1] = eb + b0;
    }
    if (j1 < P.njobs) {
      F.rbase[j1 + 1] = sa;
      F.sbase[j1 + 1] = sb;
    }
    if (lane == 0) F.rbase[0] = F.sbase[0] = 0;
  }
  __syncthreads();
  const int nrounds = F.rbase[P.njobs], nsteps = F.sbase[P.njobs];

  if (wave == kMStore) {
    // round rho's sums are complete once all 8 group wavefronts have added
    bool ok = true;
    int jb = 0;
    for (int RHO = 0; RHO < nrounds; ++RHO) {
      while (RHO >= F.rbase[jb + 1]) ++jb;   // rounds ascend: the job advances
      const MmJob &J = JOB(jb);
      const int rho = RHO - F.rbase[jb];
      const int tb = RHO & 1, nt = round_tiles(J, F.nmine[jb], rho);
      Acc *tbl = tables + tb * (TMX * CTX * 4 * 64);
      if (!mm_wait(F, [&] { return lds_read_i32(&F.tcnt[tb]) == kMW; })) {
        ok = false;
        break;
      }
      const int q = lane >> 4, c = lane & 15;
      // the job's fields, read once (kept in registers across the stores)
      int32_t *const yj = J.y32;
      const int32_t nrj = J.nrows, shj = J.sh, tmj = J.tm, nsj = J.ns;
      const MmSlice S(J, r, G);
      const int64_t half = shj > 0 ? (int64_t)1 << (shj - 1) : 0;
      // every table entry read at once, then rounded, checked and stored
      int64_t tot[TMX][CTX][4];
#pragma unroll
      for (int jj = 0; jj < TMX; ++jj)
#pragma unroll
        for (int ct = 0; ct < CTX; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            tot[jj][ct][e] = (int64_t)tbl[((jj * CTX + ct) * 4 + e) * 64 + lane];
#pragma unroll
      for (int jj = 0; jj < TMX; ++jj)
#pragma unroll
        for (int ct = 0; ct < CTX; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            tbl[((jj * CTX + ct) * 4 + e) * 64 + lane] = 0;
      bool ovf = false;
      // y = rshift_round(tot / 16, sh) (tot = 16 p): the magnitude rounded
      // half up, checked and stored
      auto put = [&](int64_t tt, int32_t *yp) {
        const int64_t v = tt >> 4;
        const int64_t m = ((v < 0 ? -v : v) + half) >> shj;
        const int64_t y = v < 0 ? -m : m;
        ovf = ovf || y > 2147483647LL || y < -2147483647LL;
        *yp = (int32_t)y;
      };
      if (nsj == 1) {
#pragma unroll
        for (int ct = 0; ct < CTX; ++ct) {
          const int tok = ct * 16 + c;
          int32_t *const yt = yj + (int64_t)tok * nrj;
#pragma unroll
          for (int jj = 0; jj < TMX; ++jj) {
            const int64_t row0 =
                ((int64_t)S.tr + (int64_t)S.tg * (rho * tmj + jj)) * kTileRows + 4 * q;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (jj < nt && ct < P.CT && tok < P.B && row0 + e < nrj)
                put(tot[jj][ct][e], yt + row0 + e);
          }
        }
      } else {
        // this slice's sums to its part of the job's partials, for
        // matmul_finish_kernel
        int64_t *const pj = J.part + (int64_t)(S.kb0 / S.nbs) * P.B * nrj;
#pragma unroll
        for (int ct = 0; ct < CTX; ++ct) {
          const int tok = ct * 16 + c;
#pragma unroll
          for (int jj = 0; jj < TMX; ++jj) {
            const int64_t row0 =
                ((int64_t)S.tr + (int64_t)S.tg * (rho * tmj + jj)) * kTileRows + 4 * q;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (jj < nt && ct < P.CT && tok < P.B && row0 + e < nrj)
                pj[(int64_t)tok * nrj + row0 + e] = tot[jj][ct][e];
          }
        }
      }
      if (ovf) mm_lds_or(&F.err, 1);
      wait_lds();
      if (lane == 0) {
        lds_write_i32(&F.tcnt[tb], 0);
        lds_write_i32(&F.tgen[tb], RHO + 2);
      }
    }
    if (!ok && lane == 0) mm_lds_or(&F.err, 4);
  } else if (wave >= kMW) {
    // loader l: steps l, l + nl, ...
    const int l = wave - kMW;
    if (l < P.nl) {
      MmCur lc;   // step s of this loader
      lc.start(F, P.njobs, JOB);
      for (int i = 0; i < l && i < nsteps; ++i) lc.next(F, P.njobs, JOB);
      int slot = l;   // s % R (l < nl < R)
      for (int s = l; s < nsteps; s += P.nl) {
        // the slot's previous step has been consumed by every group wavefront
        if (s >= P.R &&
            !mm_wait(F, [&] { return lds_read_i32(&F.done[lane & (kMW - 1)]) >= s - P.R; }))
          break;
        uint8_t *sb = ring + (size_t)slot * P.slot_bytes;
        const int kb = lc.kb0 + lc.kb;
        const int kbytes = min(1024, lc.K - kb * 1024);   // multiple of 128
        for (int tok = 0; tok < P.B; ++tok) {
          const int8_t *src = 16 * lane < kbytes
                                  ? lc.x8 + (int64_t)tok * lc.K + kb * 1024 + 16 * lane
                                  : lc.x8;   // nothing to copy: any mapped address
          dma16(src, lds_off(sb + tok * kXRow));
        }
        for (int j = 0; j < lc.nt; ++j) {
          const int64_t t = (int64_t)lc.tr + (int64_t)lc.tg * (lc.rho * lc.tm + j);
          dma4(lc.W + t * lc.tile_bytes + (int64_t)kb * kBlockBytes + 4 * lane,
               lds_off(sb + 16 * P.CT * kXRow + 256 * j));
        }
        mm_wait_vm_all();
        if (lane == 0) lds_write_i32(&F.ready[slot], s);
        for (int i = 0; i < P.nl && s + 1 + i < nsteps; ++i) lc.next(F, P.njobs, JOB);
        slot += P.nl;
        if (slot >= P.R) slot -= P.R;
      }
    }
  } else {
    const int w = wave;
    const int q = lane >> 4, c = lane & 15;
    constexpr int D = mm_depth<TMX, CTX>();
    Acc p[TMX][CTX][4];
#pragma unroll
    for (int a = 0; a < TMX; ++a)
#pragma unroll
      for (int b = 0; b < CTX; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) p[a][b][e] = 0;
    // wr[j][d]: tile j's piece of the step s with s % D == d
    uint4 wr[TMX][D];
    MmCur f, cur;   // next step to put in flight; the step being computed
    f.start(F, P.njobs, JOB);
    cur.start(F, P.njobs, JOB);
    auto fill = [&](uint4 (&slot)[TMX][D], const int d) {
      const bool any = f.RHO < nrounds;
#pragma unroll
      for (int j = 0; j < TMX; ++j) slot[j][d] = mm_issue(f, r, G, w, lane, j, any && j < f.nt);
      if (any) f.next(F, P.njobs, JOB);
    };
#pragma unroll
    for (int d = 0; d < D; ++d) fill(wr, d);
    int s = 0, slot = 0;   // slot = s % R
    int rdy = -1;          // the slot's ready word, read during the step before
    for (;;) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (s >= nsteps) goto finished;
        const int nt = cur.nt;
        if (rdy != s) mm_wait_word<false>(F, &F.ready[slot], s, lane);
        const uint8_t *sb = ring + (size_t)slot * P.slot_bytes;
        // this group's activations for the step's tokens: lane (c, q) feeds
        // token 16 ct + c, k = 128 w + 32 q + [0, 32)
        v4i bx[CTX][2];
#pragma unroll
        for (int ct = 0; ct < CTX; ++ct) {
          const int8_t *xr = (const int8_t *)sb + (16 * ct + c) * kXRow + w * 128 + 32 * q;
          const int4 u0 = *(const int4 *)xr, u1 = *(const int4 *)(xr + 16);
          bx[ct][0] = v4i{u0.x, u0.y, u0.z, u0.w};
          bx[ct][1] = v4i{u1.x, u1.y, u1.z, u1.w};
        }
        // Two or more column tiles: every product of the step first, then
        // the scales -- the MFMAs' results are read only after the last one
        // is issued, so their latency passes under the others.  One column
        // tile: tile by tile (measured faster there).
        v4i acc[TMX][CTX];
        auto products = [&](int j) {
          const uint4 wp = wr[j][d];
          const v4i a0 = {cvt_lo16(wp.x), cvt_hi16(wp.x), cvt_lo16(wp.y), cvt_hi16(wp.y)};
          const v4i a1 = {cvt_lo16(wp.z), cvt_hi16(wp.z), cvt_lo16(wp.w), cvt_hi16(wp.w)};
#pragma unroll
          for (int ct = 0; ct < CTX; ++ct) {
            if (ct < P.CT) {
              acc[j][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bx[ct][0], v4i{0, 0, 0, 0}, 0,
                                                                 0, 0);
              acc[j][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bx[ct][1], acc[j][ct], 0, 0, 0);
            }
          }
        };
        auto scales = [&](int j) {
          // this group's scales of rows 4q .. 4q+3 (row rr's 16 bytes hold
          // the block's 8 uint16 scales)
          const uint8_t *scl = sb + 16 * P.CT * kXRow + 256 * j;
          Acc m[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            m[e] = mm_scale<CTX>(*(const uint16_t *)(scl + (4 * q + e) * 16 + 2 * w));
#pragma unroll
          for (int ct = 0; ct < CTX; ++ct) {
            if (ct < P.CT) {
#pragma unroll
              for (int e = 0; e < 4; ++e) p[j][ct][e] = mm_fma(m[e], acc[j][ct][e], p[j][ct][e]);
            }
          }
        };
        if constexpr (CTX >= 2) {
#pragma unroll
          for (int j = 0; j < TMX; ++j)
            if (j < nt) products(j);
#pragma unroll
          for (int j = 0; j < TMX; ++j)
            if (j < nt) scales(j);
        } else {
#pragma unroll
          for (int j = 0; j < TMX; ++j) {
            if (j < nt) {
              products(j);
              scales(j);
            }
          }
        }
        // the next slot's ready word, read now so that its latency passes
        // under this step's remaining work
        typedef volatile __attribute__((address_space(3))) int32_t lds_i32;
        rdy = __builtin_amdgcn_readfirstlane(
            *(lds_i32 *)(lds_void_t *)&F.ready[slot + 1 == P.R ? 0 : slot + 1]);
        // refill this step's registers with the step D ahead
        fill(wr, d);
        // the slot is free: its reads were issued before this write, and
        // LDS instructions of a wavefront execute in order
        if (lane == 0) mm_lds_post(&F.done[w], s);
        if (cur.kb == cur.nblk - 1) {
          // end of round RHO: add this wavefront's sums into its table
          const int tb = cur.RHO & 1;
          Acc *tbl = tables + tb * (TMX * CTX * 4 * 64);
          mm_wait_word<true>(F, &F.tgen[tb], cur.RHO, lane);
#pragma unroll
          for (int jj = 0; jj < TMX; ++jj)
#pragma unroll
            for (int ct = 0; ct < CTX; ++ct)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                if (jj < nt && ct < P.CT)
                  mm_lds_add(&tbl[((jj * CTX + ct) * 4 + e) * 64 + lane], p[jj][ct][e]);
                p[jj][ct][e] = 0;
              }
          // the count follows the adds in this wavefront's LDS order, so the
          // store wavefront, seeing it, sees the adds: neither is waited for
          if (lane == 0) mm_lds_add_post(&F.tcnt[tb], 1);
        }
        cur.next(F, P.njobs, JOB);
        ++s;
        if (++slot == P.R) slot = 0;
      }
    }
  finished:;
  }
  __syncthreads();
  if (tid == 0) {
    const int32_t e = lds_read_i32(&F.err);
    if (e) atomicOr(P.err, e);
  }
}

// The rows of a split job: y32[tok][row] = rshift_round(sum over the ns
// slices of part / 16, sh), checked as the direct path checks it.
struct MmFinish {
  const int64_t *part;   // [ns][B][nrows]
  int32_t *y32;          // [B][nrows]
  int64_t n;             // B * nrows
  int32_t ns, sh;
};

__global__ __launch_bounds__(256) void matmul_finish_kernel(const MmFinish *fin, int32_t *err) {
  const MmFinish &F = fin[blockIdx.y];
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= F.n) return;
  int64_t tt = 0;
  for (int k = 0; k < F.ns; ++k) tt += __builtin_nontemporal_load(F.part + k * F.n + i);
  const int64_t half = F.sh > 0 ? (int64_t)1 << (F.sh - 1) : 0;
  const int64_t v = tt >> 4;
  const int64_t m = ((v < 0 ? -v : v) + half) >> F.sh;
  const int64_t y = v < 0 ? -m : m;
  if (y > 2147483647LL || y < -2147483647LL) atomicOr(err, 1);
  F.y32[i] = (int32_t)y;
}

// The jobs' records and the launch shape for B tokens: the grid (one
// workgroup per CU at most), tiles per round (TMX) and column tiles of 16
// tokens (CTX) of the kernel instance, the LDS ring and its loaders.
static hipError_t mm_setup(const MmJobSpec *jobs, int n, int32_t B, MmJob *out,
                           MmPlanCfg &c, bool split) {
  if (n < 1 || B < 1 || B > 64) return hipErrorInvalidValue;
  c.B = B;
  c.CT = (B + 15) / 16;
  int tmx = c.CT == 1 ? 4 : (c.CT == 2 ? 2 : 1);
  int dev = 0, ncu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  int maxt = 1;
  for (int j = 0; j < n; ++j) {
    MmJob &J = out[j];
    const MmJobSpec &q = jobs[j];
    J = MmJob{};
    J.W = q.w;
    J.x8 = q.x8;
    J.y32 = q.y32;
    J.tile_bytes = q.L.tile_bytes;
    J.nrows = q.nrows;
    J.ntiles = (q.nrows + kTileRows - 1) / kTileRows;
    J.NG = q.L.NG;
    J.nblk = q.L.nblk;
    J.sh = q.sh;
    J.K = q.L.K;
    J.ns = 1;
    maxt = J.ntiles > maxt ? J.ntiles : maxt;
  }
  const int G = maxt < ncu ? maxt : ncu;
  // A matrix with at most one tile per workgroup and enough tiles to give
  // every workgroup one K slice of one (a 4096-row down projection on 256
  // workgroups) is split into ns K slices when the caller has reduction
  // buffers for it (a plan): ns = 4 for up to 16 tokens, 2 for up to 32.
  const int ns_want = c.CT == 1 ? 4 : (c.CT == 2 ? 2 : 1);
  std::vector<int> per(n);
  for (int j = 0; j < n; ++j) {
    MmJob &J = out[j];
    per[j] = (J.ntiles + G - 1) / G;
    if (split && ns_want > 1 && per[j] == 1 && J.nblk % ns_want == 0 && G % ns_want == 0 &&
        J.ntiles * ns_want >= G) {
      J.ns = ns_want;
      per[j] = (J.ntiles + G / ns_want - 1) / (G / ns_want);
    }
  }
  // one tile per workgroup in every job: rounds of one tile, with the deeper
  // weight pipeline of the one-tile kernels; three a workgroup at 17..32
  // tokens (as a 12288-row matrix has on 256 workgroups): rounds of three, so
  // that one copy of a block's activations serves all three
  int maxper = 1;
  for (int j = 0; j < n; ++j) maxper = per[j] > maxper ? per[j] : maxper;
  if (maxper == 1) tmx = 1;
  else if (c.CT == 2 && maxper == 3) tmx = 3;
  const int ctxt = tmx == 4 ? 1 : (tmx >= 2 ? c.CT : (c.CT <= 2 ? c.CT : 4));
  const int table_bytes = 2 * tmx * ctxt * 4 * 64 * 8;
  c.slot_bytes = 16 * c.CT * kXRow + tmx * 256;
  const int avail = kLdsBytes - kFlagBytes - table_bytes;
  c.R = avail / c.slot_bytes;
  if (c.R > kRingMax) c.R = kRingMax;
  if (c.R < 2) return hipErrorInvalidValue;
  c.nl = c.R - 1 < kML ? c.R - 1 : kML;   // >= 1: R >= 2
  // rounds of tm tiles: as many tiles per round as the workgroups' shares
  // of the job allow, at most tmx
  for (int j = 0; j < n; ++j) out[j].tm = per[j] < tmx ? per[j] : tmx;
  c.G = G;
  c.tmx = tmx;
  c.ctxt = ctxt;
  c.lds = (size_t)kFlagBytes + table_bytes + (size_t)c.R * c.slot_bytes;
  return hipSuccess;
}

template <bool kTab>
static hipError_t mm_set_lds_limit() {
  hipError_t e = hipFuncSetAttribute((const void *)matmul_kernel<4, 1, kTab>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void *)matmul_kernel<2, 2, kTab>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void *)matmul_kernel<3, 2, kTab>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void *)matmul_kernel<1, 4, kTab>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void *)matmul_kernel<1, 1, kTab>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  if (e == hipSuccess)
    e = hipFuncSetAttribute((const void *)matmul_kernel<1, 2, kTab>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  return e;
}

template <bool kTab>
static hipError_t mm_launch(const MmParams &P, const MmPlanCfg &c, hipStream_t s) {
  // dynamic LDS beyond the default limit: allowed once per process
  static const hipError_t attr = mm_set_lds_limit<kTab>();
  if (attr != hipSuccess) return attr;
  const dim3 g(c.G), b(kMThreads);
  if (c.tmx == 4) {
    hipLaunchKernelGGL((matmul_kernel<4, 1, kTab>), g, b, c.lds, s, P);
  } else if (c.tmx == 3) {
    hipLaunchKernelGGL((matmul_kernel<3, 2, kTab>), g, b, c.lds, s, P);
  } else if (c.tmx == 2) {
    hipLaunchKernelGGL((matmul_kernel<2, 2, kTab>), g, b, c.lds, s, P);
  } else if (c.ctxt == 1) {
    hipLaunchKernelGGL((matmul_kernel<1, 1, kTab>), g, b, c.lds, s, P);
  } else if (c.ctxt == 2) {
    hipLaunchKernelGGL((matmul_kernel<1, 2, kTab>), g, b, c.lds, s, P);
  } else {
    hipLaunchKernelGGL((matmul_kernel<1, 4, kTab>), g, b, c.lds, s, P);
  }
  return hipGetLastError();
}

static void mm_params(MmParams &P, int n, const MmPlanCfg &c, int32_t *err) {
  P.njobs = n;
  P.B = c.B;
  P.CT = c.CT;
  P.R = c.R;
  P.nl = c.nl;
  P.slot_bytes = c.slot_bytes;
  P.err = err;
}

}  // namespace

size_t matmul_job_bytes() { return sizeof(MmJob); }

hipError_t matmul_plan_prepare(const MmJobSpec *jobs, int n, int32_t B, void *table,
                               MmPlanCfg *cfg, int32_t *ns) {
  if (n < 1 || n > kMmPlanJobs || !table || !cfg || !ns) return hipErrorInvalidValue;
  const hipError_t e = mm_setup(jobs, n, B, (MmJob *)table, *cfg, true);
  for (int j = 0; e == hipSuccess && j < n; ++j) ns[j] = ((const MmJob *)table)[j].ns;
  return e;
}

void matmul_plan_bind(void *table, int j, int64_t *part) { ((MmJob *)table)[j].part = part; }

size_t matmul_finish_bytes() { return sizeof(MmFinish); }

int matmul_finish_prepare(const void *table, int n, int32_t B, void *fin) {
  int nf = 0;
  for (int j = 0; j < n; ++j) {
    const MmJob &J = ((const MmJob *)table)[j];
    if (J.ns <= 1) continue;
    MmFinish &f = ((MmFinish *)fin)[nf++];
    f.part = J.part;
    f.y32 = J.y32;
    f.n = (int64_t)B * J.nrows;
    f.ns = J.ns;
    f.sh = J.sh;
  }
  return nf;
}

hipError_t launch_matmul_finish(const void *d_fin, int nf, int64_t max_n, int32_t *err,
                                hipStream_t s) {
  if (nf < 1) return hipSuccess;
  const dim3 g((unsigned)((max_n + 255) / 256), (unsigned)nf);
  hipLaunchKernelGGL(matmul_finish_kernel, g, dim3(256), 0, s, (const MmFinish *)d_fin, err);
  return hipGetLastError();
}

hipError_t launch_matmul_plan(const void *d_table, int n, const MmPlanCfg &cfg, int32_t *err,
                              hipStream_t s) {
  if (n < 1 || n > kMmPlanJobs || !d_table) return hipErrorInvalidValue;
  MmParams P{};
  mm_params(P, n, cfg, err);
  P.tab = (const MmJob *)d_table;
  return mm_launch<true>(P, cfg, s);
}

hipError_t launch_matmul_multi(const MmJobSpec *jobs, int n, int32_t B, int32_t *err,
                               hipStream_t s) {
  if (n < 1 || n > kMmJobs) return hipErrorInvalidValue;
  MmParams P{};
  MmPlanCfg c{};
  hipError_t e = mm_setup(jobs, n, B, P.job, c, false);
  if (e != hipSuccess) return e;
  mm_params(P, n, c, err);
  return mm_launch<false>(P, c, s);
}

hipError_t launch_matmul(const uint8_t *w, int32_t nrows, const Layout &L, int32_t sh,
                         const int8_t *x8, int32_t B, int32_t *y32, int32_t *err,
                         hipStream_t s) {
  const MmJobSpec j{w, nrows, L, sh, x8, y32};
  return launch_matmul_multi(&j, 1, B, err, s);
}

}  // namespace w4a8
