// Persistent decode-step kernel (W4A8_PLAN_PERSISTENT) for gfx950.
//
// One launch runs every site of a plan, one workgroup per CU of
// 12 wavefronts with three roles, which meet only through LDS flags -- no
// workgroup barrier while the plan runs:
//
//  * 8 weight wavefronts stream the weights and do the dot products.  The
//    weight blocks this CU owns over the whole plan form one fixed sequence
//    (its tiles of site 0, then of site 1, ...; 8448-byte scale blocks
//    within a tile), dealt round-robin to the 8 wavefronts.  Each wavefront
//    holds its next two blocks in two register sets, A and B, and refills a
//    set as soon as it has consumed it -- also when the next block belongs
//    to a later site, since weights never depend on an activation.  Every
//    refill is the same 9 buffer loads (out of range, so without a memory
//    access, past the end of the sequence), and a weight wavefront makes no
//    other global access, so the compiler's count of its outstanding loads
//    is exact on every path.  (Its waits are not minimal: at the loop head
//    the first set's dot product waits for both sets.  Loads and waits of
//    our own in inline assembly, one set at a time, measured slower.)  At
//    its first block of a site it waits only for that site's activations
//    (an LDS flag), never for the other wavefronts.
//  * 3 prologue wavefronts compute each site's activations (RMSNorm, DYNQ8:
//    x8, e_x and the offset corrections) ahead of the weight wavefronts,
//    into a ring of 8 LDS buffers; a buffer is reused once every weight
//    wavefront has moved past the site that used it.
//  * 1 control wavefront stores the outputs, which the wavefront completing
//    a tile stages in LDS, and at a fenced site waits until every workgroup
//    has stored its outputs of all earlier sites (one flag per workgroup)
//    before the prologue wavefronts may read that site's activations.  At a
//    site whose input is the site it has just stored, it computes a fourth
//    share of the prologue (ctrl_assists).
//
// A tile's 16 rows are complete when every weight wavefront holding one of
// its blocks has added its partial sums into an LDS slot; the wavefront
// that completes the count rounds, checks and applies the epilogue.  The LDS
// flags are inline assembly (the compiler's own LDS synchronisation makes a
// wavefront wait for all of its outstanding loads).  Data crossing a site
// boundary (outputs, activation vectors, flags) moves with agent-coherent
// accesses (sc1), so no cache-wide writeback or invalidation is needed.
// Every result is bit-exact with the reference's integer law
// (ref/w4a8_ref.py:254-289, fixedpoint.py:24-75, layer_fixed.py:1242-1278
// and the epilogues of gen_layer_script.py:1397-1433, seq_model.py:1027-1050).
#include <hip/hip_ext.h>

#include "w4a8_device.h"
#include "w4a8_topk_device.h"

namespace w4a8 {

namespace {

constexpr int kCW = 8;                      // weight wavefronts 0..7
constexpr int kCtrl = kCW;                  // the control wavefront
constexpr int kPW = 3;                      // prologue wavefronts
constexpr int kPW0 = kCW + 1;               // ... 9..11
constexpr int kThreads = (kPW0 + kPW) * 64; // 768
constexpr int kPR = kPW + 1;                // ready flags per buffer: the prologue
                                            // wavefronts and the control wavefront
static_assert((kPR & (kPR - 1)) == 0, "a lane picks its flag with a mask");
constexpr int kNB = 8;                      // activation buffers (a power of 2)
constexpr int kExpX8 = 1;                   // a prologue's exports: x8 and e_x ...
constexpr int kExpXn = 2;                   // ... the RMSNorm output
constexpr int kXloOff = kKMax;              // int32 corrections after x8
constexpr int kXB = kKMax + kKMax / 8;      // x8 + corrections of one site
constexpr int kTSlots = 32;                 // tiles being reduced at once
constexpr int kChunk = 64 * 8;              // int16 elements per prologue chunk
constexpr int kPC = (kKMax / kChunk + kPW - 1) / kPW;             // chunks per wavefront
constexpr int kPN = (kStreamNormKMax / kChunk + kPW - 1) / kPW;   // RMSNorm chunks
constexpr int kPX = (kKMax / 1024 + kPW - 1) / kPW;               // int8 chunks (1 KiB)
constexpr uint32_t kGridSpin = 1u << 18;    // polls before a grid wait gives up
constexpr int kBufDword3 = 0x00020000;      // raw buffer, 32-bit data format
constexpr int kAuxSc1 = 16;                 // buffer-load cache policy: agent-coherent

static_assert(kKMax % kChunk == 0 && kStreamNormKMax % kChunk == 0, "whole chunks");
static_assert((kTSlots & (kTSlots - 1)) == 0, "slot index is a mask");
static_assert(kXB % 16 == 0, "buffers stay 16-byte aligned");

// The site table is read-only for the whole launch.  Read through the
// constant address space, every (uniform) field load is a scalar load, also
// after LDS waits, so weight wavefronts never issue a vector load of their
// own besides the weight loads.
typedef const __attribute__((address_space(4))) GemvParams CSite;
typedef const __attribute__((address_space(4))) GemvJob CJob;

struct __align__(16) Lds {
  int8_t x[kNB][kXB];               // x8 and corrections of site s in x[s % kNB]
  int64_t tv[kTSlots][kTileRows];   // partial sums, then staged outputs
  int32_t tcnt[kTSlots];            // contributions added to the slot
  int32_t tgen[kTSlots];            // tile number the slot is open for
  int32_t tready[kTSlots];          // tile number + 1 once its outputs are staged
  int32_t ready[kNB][kPR];          // per prologue wavefront (and the control wavefront
                                    // last): the site whose activations it has written
                                    // into the buffer (-1: none)
  int32_t ex[kNB];                  // ... and its e_x
  int32_t wsite[kCW];               // site each weight wavefront works on (nsites: done)
  int32_t gridok;                   // last fenced site whose grid-wide wait has passed
  int32_t served;                   // last site whose outputs the control wavefront stored
  int32_t xdone;                    // last site whose x8 / e_x the control wavefront exported
  int16_t pairv[kPairTiles][kTileRows];  // paired site: job 0's outputs of this CU's tiles
  int16_t prod[kTileRows];          // ... and one tile's EMUL32 products
  int32_t psync[kPW];               // prologue wavefronts' barrier phases
  int32_t psync4[kPR];              // ... with the control wavefront (site-numbered phases)
  int32_t abort;                    // set by the first LDS wait that gives up
  int32_t err;                      // error bits found inside the workgroup
  uint16_t rsqrt[512];
  uint16_t sig[264];
  int64_t pss[kPR];                 // prologue partial sums of squares
  int32_t pmx[kPR];                 // prologue partial maxima
  uint64_t best;                    // argmax key of the head's rows seen here (0: none)
  uint64_t tkbuf[128];              // TOPK-32 head: the scan's key buffer ...
  int32_t tkrows[tk::kTkRows];      // ... and its chunk's values (prologue wavefront 0)
};

// The workgroup's LDS block.
__shared__ Lds g_lds;

// a pointer argument of a non-inlined function, made wavefront-uniform
__device__ __forceinline__ void *uniform_ptr(const void *p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return (void *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// This lane's index, computed afresh where it is needed (v_mbcnt, in an asm
// statement the compiler can neither hoist nor merge), so that no register
// holds the thread index across the roles' loops: held, it was spilled to
// scratch in the dependent-site instances, and the reload sat in the weight
// loop.
__device__ __forceinline__ int lane_now() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// ---------------------------------------------------------------------------
// LDS synchronisation
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// lane l copies 16 bytes from src (its own address, agent-coherent) to LDS
// lds_base + 16 * l; lds_base must be uniform
__device__ __forceinline__ void copy16_sc1(const void *src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1"
               :: "v"(src), "s"(lds_base) : "memory", "m0");
}

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
__device__ __forceinline__ void lds_wait_eq(Lds &L, const int32_t *p, int v, int lane,
                                            uint32_t lspin) {
  if (lane == 0) {
    uint32_t n = 0;
    for (;;) {
      const int32_t cur = lds_read_i32(p);
      if ((kAtLeast ? cur >= v : cur == v) || lds_read_i32(&L.abort) != 0) break;
      __builtin_amdgcn_s_sleep(1);
      if (++n > lspin) {
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
  int i, b;   // ... as tile and block: j = i * nblk + b (kept by additions: a
              // division per block, in scalar code shared by the CU's
              // wavefronts, cost a weight wavefront more time than its dot)
  int kt0;    // CU-local number of the site's first tile
  int nb;     // blocks of the site on this CU
  int ntl;    // tiles of the site on this CU
  int nblk;   // scale blocks per tile
  int first;  // first global tile of the site on this CU
  int ng;     // scale groups per row (the site's NG)
  int tbytes; // bytes per tile
  int job;    // the job of tile i (a site's jobs are runs of tiles, and t only grows)
  int jend;   // ... the first tile past it
  uint64_t jbase;   // ... and its weights' address less its first tile's offset
  int jtile0, jrows;   // ... its first tile and rows
  int jepi;   // ... and its epilogue: epi | sh << 8 | p0 << 16 (kept here, so a
              // tile's epilogue reads no table entry, which may have left the
              // scalar cache since the tile's first block)
};

// Workgroup r's first tile of site P and its number of tiles there, without
// a division (r and tile_rot lie in [0, G))
__device__ __forceinline__ int site_first(CSite &P, int r, int G) {
  const int f = r + P.tile_rot;
  return f >= G ? f - G : f;
}
__device__ __forceinline__ int site_ntl(CSite &P, int first) {
  return P.tiles_q + (first < P.tiles_r ? 1 : 0);
}
// s % G for a site number (a plan has few more sites than workgroups)
__device__ __forceinline__ int site_owner(int s, int G) {
  while (s >= G) s -= G;
  return s;
}

__device__ __forceinline__ void cur_load_site(CSite *sites, int r, int G, Cursor &c) {
  CSite &P = sites[c.s];
  c.first = site_first(P, r, G);
  c.ntl = site_ntl(P, c.first);
  c.nblk = P.nblk;
  c.nb = c.ntl * c.nblk;
  c.ng = P.NG;
  c.tbytes = (int)P.tile_bytes;
}

// The job of tile i (global tile first + i * G), found from the cursor's
// job on (from job 0 when `fresh`): the table is read only when the tile
// leaves the job, so the weight loop's block addresses take no table reads.
__device__ __forceinline__ void cur_job(CSite *sites, int G, Cursor &c, bool fresh) {
  CSite &P = sites[c.s];
  const int t = c.first + c.i * G;
  if (!fresh && t < c.jend) return;
  int j = fresh ? 0 : c.job;
  while (j + 1 < P.njobs && t >= P.tile0[j + 1]) ++j;
  c.job = j;
  c.jend = j + 1 < P.njobs ? P.tile0[j + 1] : 0x7fffffff;
  CJob &J = P.job[j];
  c.jbase = (uint64_t)(uintptr_t)J.w - (uint64_t)(int64_t)J.tile0 * (uint64_t)(int64_t)c.tbytes;
  c.jtile0 = J.tile0;
  c.jrows = J.nrows;
  c.jepi = (J.epi & 0xFF) | ((J.sh & 0xFF) << 8) | (int)((uint32_t)J.p0 << 16);
}

// (i, b) of block j, from i = 0 (j is below a few nblk here)
__device__ __forceinline__ void cur_split(Cursor &c) {
  c.i = 0;
  c.b = c.j;
  while (c.b >= c.nblk && c.nblk > 0) {
    c.b -= c.nblk;
    ++c.i;
  }
}

// move forward until block j lies in site s (or past the last site)
__device__ __forceinline__ void cur_settle(CSite *sites, int nsites, int r, int G, Cursor &c) {
  if (c.s < nsites && c.j >= c.nb) {
    while (c.s < nsites && c.j >= c.nb) {
      c.j -= c.nb;
      c.kt0 += c.ntl;
      ++c.s;
      if (c.s < nsites) cur_load_site(sites, r, G, c);
    }
    cur_split(c);
    if (c.s < nsites) cur_job(sites, G, c, true);
  }
}

__device__ __forceinline__ void cur_init(CSite *sites, int nsites, int r, int G, int j0,
                                         Cursor &c) {
  c.s = 0;
  c.j = j0;
  c.kt0 = 0;
  c.nb = c.ntl = c.nblk = c.first = c.ng = c.tbytes = c.job = c.jend = 0;
  c.jtile0 = c.jrows = c.jepi = 0;
  c.jbase = 0;
  if (nsites > 0) cur_load_site(sites, r, G, c);
  cur_split(c);
  if (nsites > 0 && c.j < c.nb) cur_job(sites, G, c, true);
  cur_settle(sites, nsites, r, G, c);
}

__device__ __forceinline__ void cur_next(CSite *sites, int nsites, int r, int G, Cursor &c) {
  c.j += kCW;
  c.b += kCW;
  while (c.b >= c.nblk && c.nblk > 0) {
    c.b -= c.nblk;
    ++c.i;
  }
  if (c.s < nsites && c.j >= c.nb) cur_settle(sites, nsites, r, G, c);
  else if (c.s < nsites) cur_job(sites, G, c, false);
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
    const uint32_t t = (uint32_t)(c.first + c.i * G);
    bb = (const uint8_t *)(uintptr_t)(c.jbase + (uint64_t)t * (uint32_t)c.tbytes +
                                      (uint64_t)(uint32_t)(c.b * kBlockBytes));
    len = kScaleChunk + groups_in(c.ng, c.b) * kGroupChunk;
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

// ------------------------------------------------------------- tiles
// Add this wavefront's share of tile kt; true if it completed the tile.
__device__ __forceinline__ bool tile_add(Lds &L, int kt, int64_t p, int contributors, uint32_t lspin,
                                         int lane) {
  const int slot = kt & (kTSlots - 1);
  lds_wait_eq(L, &L.tgen[slot], kt, lane, lspin);
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
// (the job's epi, sh and p0 packed as in Cursor::jepi, and its rows)
__device__ __forceinline__ void tile_epilogue(Lds &L, int kt, int jepi, int nrows, int tl,
                                              int e_x, int lane) {
  const int slot = kt & (kTSlots - 1);
  const int epi = jepi & 0xFF, sh = (jepi >> 8) & 0xFF, p0 = jepi >> 16;
  const bool argmax = epi == EPI_ARGMAX;
  if (lane < kTileRows) {
    const int64_t tot = L.tv[slot][lane];
    const int row = tl * kTileRows + lane;
    int64_t outv = 0;
    if (row < nrows) {
      const int64_t y = rshr64(tot >> 4, sh);   // tot is 16 * p exactly
      if (y > 2147483647LL || y < -2147483647LL) lds_or_i32(&L.err, 1);
      const int shift = p0 - e_x;
      switch (epi) {
        case EPI_Y32: outv = y; break;
        case EPI_MOVY_I16: outv = clamp64(movy_shift(y, shift), -32768, 32767); break;
        case EPI_MOVY_P32:
          outv = clamp64(movy_shift(y, shift), -2147483648LL, 2147483647LL);
          break;
        case EPI_SILU32: outv = silu32(y, shift, L.sig); break;
        case EPI_SHIFT_I64: outv = movy_shift(y, shift); break;
        case EPI_TOPK: outv = y; break;   // raw y32, as for the argmax
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
// A residual-ADD tile's stores: MOVY int16 into out (when set), and the
// block's residual ALU ADD clip16(res + that) into res_out
// (gen_layer_script.py:1399-1400), whose values replace the tile's in LDS
// for the stamped words.  Out of line: the other epilogues' store path is
// the control wavefront's critical path in a chained step.
__device__ __noinline__ void serve_residual(Lds &L, CJob &J, int slot, int t, int lane) {
  if (lane < kTileRows) {
    const int64_t v = L.tv[slot][lane];
    const int row = (t - J.tile0) * kTileRows + lane;
    if (row < J.nrows) {
      if (J.out) store_coherent((int16_t *)J.out + row, (int16_t)v);
      const int64_t rv = clamp64(
          v + __hip_atomic_load(J.res + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
          -32768, 32767);
      store_coherent(J.res_out + row, (int16_t)rv);
      L.tv[slot][lane] = rv;
    }
  }
  wait_lds();
}

// Store the outputs of this CU's tiles of site P (tile numbers kt0, ...), and
// for a job read through stamped words also the words (lanes 0..7: rows
// 2l, 2l+1 of the tile with `stamp`; each an 8-byte store, which lands
// whole, so a reader that sees the stamp sees the rows).
// Argmax tiles stage nothing: their slot is freed by the wavefront that
// completes them, which is waited for here too, so that no wavefront still
// reads this site's activations once this returns.
template <bool kDep>
__device__ __forceinline__ void ctrl_serve(CSite &P, Lds &L, int kt0, int r, int G, int lane,
                                           uint32_t stamp, uint32_t lspin) {
  const int first = site_first(P, r, G);
  // the job of tile t, found from the last one on (t only grows), and the
  // fields its tiles' stores need, read from the table only when the job
  // changes: a table read on every tile put its latency before every store
  int j = -1, jend = 0, epi = 0, jt0 = 0, nrows = 0;
  void *out = nullptr;
  uint64_t *stamped = nullptr;
  bool add = false;
  for (int i = 0, t = first; t < P.total_tiles; ++i, t += G) {
    if (t >= jend) {
      if (j < 0) j = 0;
      while (j + 1 < P.njobs && t >= P.tile0[j + 1]) ++j;
      CJob &Jn = P.job[j];
      jend = j + 1 < P.njobs ? P.tile0[j + 1] : 0x7fffffff;
      epi = Jn.epi;
      jt0 = Jn.tile0;
      nrows = Jn.nrows;
      out = Jn.out;
      stamped = Jn.stamped;
      // a residual-ADD job reaches this kernel as EPI_MOVY_I16 with res_out
      add = Jn.res_out != nullptr;
    }
    CJob &J = P.job[j];
    const int kt = kt0 + i, slot = kt & (kTSlots - 1);
    if (epi == EPI_ARGMAX) {
      // later argmax tiles may have reused and freed the slot since
      lds_wait_eq<true>(L, &L.tgen[slot], kt + kTSlots, lane, lspin);
      continue;
    }
    lds_wait_eq(L, &L.tready[slot], kt + 1, lane, lspin);
    if (add) serve_residual(L, J, slot, t, lane);
    if (kDep && stamped && lane < kTileRows / 2) {
      // rows 2l and 2l + 1 (int16 epilogues); nrows is even
      const int row = (t - jt0) * kTileRows + 2 * lane;
      const uint32_t lo = (uint32_t)(uint16_t)(int16_t)L.tv[slot][2 * lane];
      const uint32_t hi = (uint32_t)(uint16_t)(int16_t)L.tv[slot][2 * lane + 1];
      if (row < nrows)
        store_coherent(stamped + row / 2, (uint64_t)(lo | (hi << 16)) | ((uint64_t)stamp << 32));
    }
    if (lane < kTileRows) {
      const int64_t v = L.tv[slot][lane];
      const int row = (t - jt0) * kTileRows + lane;
      if (row < nrows && !add) {
        switch (epi) {
          case EPI_MOVY_I16:
          case EPI_SILU32: store_coherent((int16_t *)out + row, (int16_t)v); break;
          case EPI_SHIFT_I64: store_coherent((int64_t *)out + row, v); break;
          case EPI_TOPK:
            // {y32, stamp}: an 8-byte store lands whole, so the scan, seeing
            // this launch's stamp, sees the value
            store_coherent((uint64_t *)out + row,
                           (uint64_t)(uint32_t)(int32_t)v | ((uint64_t)stamp << 32));
            break;
          default: store_coherent((int32_t *)out + row, (int32_t)v); break;
        }
      }
      L.tv[slot][lane] = 0;
      if (kDep && P.prod_stamped) {
        // a paired site: this CU's tiles of job 0 come first (npair of
        // them), then the same tiles of job 1; ALU EMUL32 at p0 = 12
        // (gen_layer_script.py:1414-1418) of the two, as job 1's are stored
        const int npair = P.tiles_q >> 1;   // total_tiles = 2 * npair * G
        if (i < npair) {
          L.pairv[i][lane] = (int16_t)v;
        } else {
          const int64_t pr = rshr64(v * (int64_t)L.pairv[i - npair][lane], kEmulP0);
          L.prod[lane] = (int16_t)clamp64(pr, -32768, 32767);
        }
      }
    }
    if (kDep && P.prod_stamped && i >= (P.tiles_q >> 1) && lane < kTileRows / 2) {
      wait_lds();
      const int row = (t - jt0) * kTileRows + 2 * lane;
      const uint32_t lo = (uint32_t)(uint16_t)L.prod[2 * lane];
      const uint32_t hi = (uint32_t)(uint16_t)L.prod[2 * lane + 1];
      store_coherent(P.prod_stamped + row / 2, (uint64_t)(lo | (hi << 16)) | ((uint64_t)stamp << 32));
    }
    if (lane == 0) {
      lds_write_i32(&L.tcnt[slot], 0);
      lds_write_i32(&L.tgen[slot], kt + kTSlots);
    }
  }
}

// all G workgroups have stored flag value >= v (bounded; bit 1 of err)
__device__ __forceinline__ void grid_wait(uint32_t *flags, int G, uint32_t v, int lane,
                                          int32_t *err, uint32_t gspin) {
  uint32_t n = 0;
  for (;;) {
    bool ok = true;
    for (int i = lane; i < G; i += 64)
      ok = ok && __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= v;
    if (__all(ok)) break;
    __builtin_amdgcn_s_sleep(1);
    if (++n > gspin) {
      if (lane == 0) atomicOr(err, 2);
      break;
    }
  }
}


// ------------------------------------------------------------- prologue
// The prologue wavefronts' barrier state: its phase, and whether every wait
// so far ended.  A value type, passed in and out of the staged prologue's
// (non-inlined) function, so it stays in registers.
struct PSync {
  int32_t phase;
  int32_t ok;
};

// barrier of the 3 prologue wavefronts only (bounded), through L.psync;
// with NP = kPR also the control wavefront, through L.psync4, whose phases
// the caller numbers by site (the control wavefront takes part in some
// sites' prologues only)
template <int NP = kPW>
__device__ __forceinline__ void psync(Lds &L, PSync &ps, int pw, int lane, uint32_t lspin) {
  int32_t *f = NP == kPW ? L.psync : L.psync4;
  ++ps.phase;
  wait_lds();
  if (lane == 0) lds_write_i32(&f[pw], ps.phase);
  bool done = false;
  for (uint32_t n = 0; n < lspin && !done; ++n)
    done = __all(lds_read_i32(&f[lane % NP]) >= ps.phase);
  ps.ok = ps.ok && done;
}

// Bring site P's table entry into the scalar cache (one load per 64-byte
// line), so that the waits and the epilogue at the site's fence do not each
// miss on it.
__device__ __forceinline__ void touch_site(CSite *P) {
  typedef const __attribute__((address_space(4))) int32_t CInt;
  CInt *q = (CInt *)P;
  int32_t acc = 0;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(GemvParams) / 4); i += 16) acc ^= q[i];
  asm volatile("" ::"s"(acc));
}

// One 16-byte piece of a vector through a buffer whose range ends with the
// vector: lanes past it read zero.  Agent-coherent, since an earlier site on
// another CU may have written it.
__device__ __forceinline__ int4 vec_load(__amdgpu_buffer_rsrc_t rs, int off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kAuxSc1);
  return make_int4((int)v.x, (int)v.y, (int)v.z, (int)v.w);
}

// One prologue wavefront's share of a site's inputs, in registers: int16 x
// in chunks g = pw, pw + 3, ... of 512 elements (lane l holds elements
// 8l..8l+7 of a chunk, so the 4 lanes of a DPP quad hold 32 consecutive
// elements -- one (group, k-quarter) of the weight layout), the RMSNorm
// weights and the int32 second factor of PRO_EMUL_DYNQ8 alike; for int8 x
// (PRO_X8), 1 KiB chunks of 16 bytes per lane.
// NC chunks per wavefront: kPC for any K, or kPS for a site read through
// stamped words with K <= kStampKSmall (see small_prologue).
template <int NC>
struct ProXN {
  int4 pc[NC];
  int4 wv[kPN];
  int4 x2[NC];   // PRO_EMUL_DYNQ8: the second factor of half the chunks at a time
};
typedef ProXN<kPC> ProX;
constexpr int kPS = kPN;                        // chunks per wavefront for K <= ...
constexpr int kStampKSmall = kPS * kPW * kChunk;   // ... 4608
constexpr int kPC2 = kPC / 2;   // chunks per half of the second factor
static_assert(kPC % 2 == 0, "the second factor is loaded in two halves");

// The second factor of chunks h * kPC2 .. + kPC2 (PRO_EMUL_DYNQ8) into X.x2.
__device__ __forceinline__ void pro_issue_x2(ProX &X, CSite &P, int half, int pw, int lane) {
  const int x2len = P.pro == PRO_EMUL_DYNQ8 ? 4 * P.K : 0;
  const __amdgpu_buffer_rsrc_t r2 =
      __builtin_amdgcn_make_buffer_rsrc((void *)P.x2, (short)0, x2len, kBufDword3);
#pragma unroll
  for (int i = 0; i < kPC2; ++i) {
    const int off = (((half * kPC2 + i) * kPW + pw) * kChunk + lane * 8) * 4;
    X.x2[2 * i] = vec_load(r2, off);
    X.x2[2 * i + 1] = vec_load(r2, off + 16);
  }
}

// Put site P's inputs for prologue wavefront pw in flight: always the same
// buffer loads (out of range where there is nothing to load), all issued
// before any is waited for.
template <bool kDep>
__device__ __forceinline__ void pro_issue(ProX &X, CSite &P, int pw, int lane) {
  const int K = P.K;
  const bool x8 = P.pro == PRO_X8;
  const int xlen = x8 ? K : 2 * K;
  const int wlen = P.pro == PRO_RMSNORM_DYNQ8 ? 2 * K : 0;
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void *)P.x, (short)0, xlen, kBufDword3);
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void *)P.norm_w, (short)0, wlen, kBufDword3);
#pragma unroll
  for (int c = 0; c < kPC; ++c) {
    const int off = x8 ? (c < kPX ? (c * kPW + pw) * 1024 + lane * 16 : 1 << 30)
                       : ((c * kPW + pw) * kChunk + lane * 8) * 2;
    X.pc[c] = vec_load(rx, off);
  }
#pragma unroll
  for (int c = 0; c < kPN; ++c) X.wv[c] = vec_load(rw, ((c * kPW + pw) * kChunk + lane * 8) * 2);
  if (kDep) pro_issue_x2(X, P, 0, pw, lane);
}

// Site P's x through the stamped words of site P.stamp_src (stamp): every
// lane's chunks as in pro_issue (lane l of chunk c: elements 8l..8l+7, four
// words in two 16-byte loads, into X.pc[c] and X.x2[c]), reloaded until every
// word of the wavefront carries the stamp; then X.pc[c] holds the chunk's
// 8 int16.  The RMSNorm weights are loaded first, as in pro_issue.
// Bounded: false if the words never all arrived (err bit 1).
template <int NC, int NP = kPW>
__device__ __forceinline__ bool pro_issue_stamped(ProXN<NC> &X, CSite &P, int K, int pro,
                                                  uint32_t stamp, int pw, int lane, int32_t *err,
                                                  uint32_t gspin) {
  const int wlen = pro == PRO_RMSNORM_DYNQ8 ? 2 * K : 0;
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void *)P.norm_w, (short)0, wlen, kBufDword3);
#pragma unroll
  for (int c = 0; c < kPN; ++c) X.wv[c] = vec_load(rw, ((c * NP + pw) * kChunk + lane * 8) * 2);
  // words past K are out of the buffer's range: they read as zero, so a
  // lane whose 8 elements lie past K (K % 8 == 0) takes them as arrived --
  // per lane, since K need not fill a chunk
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void *)P.x_stamped, (short)0, 4 * K, kBufDword3);
  bool ok = false;
  for (uint32_t n = 0; n < gspin && !ok; ++n) {
    if (n > 0) __builtin_amdgcn_s_sleep(2);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int off = ((c * NP + pw) * kChunk + lane * 8) * 4;
      X.pc[c] = vec_load(rx, off);
      X.x2[c] = vec_load(rx, off + 16);
    }
    // every word checked with bitwise operations, no branch: a
    // short-circuit check compiled to a cascade of exec-mask branches, one
    // per chunk, that lengthened every poll (chained step 1.351 -> 1.300
    // ms, FFN blocks in layer order 0.630 -> 0.623 ms)
    uint32_t bad = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const bool past = (c * NP + pw) * kChunk + lane * 8 >= K;
      const uint32_t d = ((uint32_t)X.pc[c].y ^ stamp) | ((uint32_t)X.pc[c].w ^ stamp) |
                         ((uint32_t)X.x2[c].y ^ stamp) | ((uint32_t)X.x2[c].w ^ stamp);
      bad |= past ? 0u : d;
    }
    ok = __all(bad == 0);
  }
  if (!ok && lane == 0) atomicOr(err, 2);
  // (X.x2 is left as loaded: a site read through stamped words is a DYNQ8
  // or RMSNorm site, never the EMUL32 one whose second factor X.x2 holds,
  // and clearing it took 32 moves per site: chained step 1.351 -> 1.344 ms)
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    X.pc[c] = make_int4(X.pc[c].x, X.pc[c].z, X.x2[c].x, X.x2[c].z);
  }
  return ok;
}

// 8 bytes into the staging area, visible to every CU once waited for
__device__ __forceinline__ void stage_u64(int8_t *p, uint32_t lo, uint32_t hi) {
  store_coherent((uint64_t *)p, (uint64_t)lo | ((uint64_t)hi << 32));
}

// Where a prologue puts x8 and the offset corrections: the site's staging
// area in global memory (agent-coherent stores, kLds false) or this CU's
// own LDS buffer (kLds true); the layout is the same.
template <bool kLds>
__device__ __forceinline__ void put_x8(int8_t *base, int off, uint32_t lo, uint32_t hi) {
  if (kLds) *(uint2 *)(base + off) = make_uint2(lo, hi);
  else stage_u64(base + off, lo, hi);
}
template <bool kLds>
__device__ __forceinline__ void put_corr(int8_t *base, int i, int32_t v) {
  int32_t *xlo = (int32_t *)(base + kXloOff);
  if (kLds) xlo[i] = v;
  else store_coherent(&xlo[i], v);
}

// Packed 16-bit helpers for the prologue: two int16 of a 32-bit word per
// instruction (v_pk_* integer operations; exact integer arithmetic).
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// |v| of both int16 of w, as uint16 (|-32768| = 32768)
__device__ __forceinline__ u16x2 abs2(int32_t w) {
  const u16x2 u = __builtin_bit_cast(u16x2, w);
  const u16x2 n = (u16x2)(0) - u;
  return __builtin_bit_cast(
      u16x2, __builtin_elementwise_max(__builtin_bit_cast(s16x2, u), __builtin_bit_cast(s16x2, n)));
}

// DYNQ8 of both int16 of w at exponent e (half = (1 << e) >> 1, e <= 9):
// clip(rshift_round(v, e), -127, 127) in each 16-bit half (its low byte is
// the int8)
__device__ __forceinline__ uint32_t dynq2(int32_t w, u16x2 half, u16x2 e2) {
  u16x2 q = (abs2(w) + half) >> e2;   // <= 32768 + 256: no wrap
  q = __builtin_elementwise_min(q, (u16x2)(127));
  const u16x2 sgn = __builtin_bit_cast(u16x2, __builtin_bit_cast(s16x2, w) >> (s16x2)(15));
  return __builtin_bit_cast(uint32_t, (q ^ sgn) - sgn);
}

// the low bytes of the four int16 in (a, b) as one word: a.lo, a.hi, b.lo, b.hi
__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x06040200u);
}

// The prologue of site P by the 3 prologue wavefronts (pw = 0..2; ps is
// their barrier) from the inputs in X: x8 and the offset corrections into
// `out` (put_x8 / put_corr), and the site's exports named by `exports` (kExpX8: x8 and
// e_x; kExpXn: the RMSNorm
// output); returns e_x.  Chunks past K are skipped.
template <bool kLds, bool kDep, int NC = kPC, int NP = kPW>
__device__ __forceinline__ int group_prologue(CSite &P, int K, int pro, Lds &L, int8_t *out,
                                              int exports, int pw, int lane, PSync &ps,
                                              ProXN<NC> &X, uint32_t lspin) {
  // (the int8-input and EMUL32 variants only with every chunk: a site read
  // through stamped words is a DYNQ8 or RMSNorm site)
  // kAll: every chunk is computed, without a branch (its inputs past K read
  // as zero), so that the compiler interleaves the chunks' instructions; only
  // in LDS, where chunks past K < 4608 land in the buffer's unused room, and
  // never with x8 exports (kExpX8), which go to global memory
  static_assert(NC != kPC || NP == kPW, "every chunk: the prologue wavefronts only");
  constexpr bool kAll = kLds && NC <= kPS;
  constexpr int kRN = NC < kPN ? NC : kPN;   // RMSNorm chunks held
  if constexpr (NC == kPC) if (pro == PRO_X8) {
#pragma unroll
    for (int c = 0; c < kPX; ++c) {
      const int off = (c * NP + pw) * 1024 + lane * 16;
      if ((c * NP + pw) * 1024 < K) {
        const int4 v = X.pc[c];
        // -8 * sum of the x8 met by the offset-form low nibbles of a
        // 32-byte (group, quarter): bytes 0-3 and 8-11 of each lane's 16,
        // lane pairs
        int t = __builtin_amdgcn_sdot4(v.x, 0x01010101, 0, false);
        t = __builtin_amdgcn_sdot4(v.z, 0x01010101, t, false);
        t += __builtin_amdgcn_update_dpp(0, t, 0xB1, 0xF, 0xF, false);
        if (off < K) {
          put_x8<kLds>(out, off, (uint32_t)v.x, (uint32_t)v.y);
          put_x8<kLds>(out, off + 8, (uint32_t)v.z, (uint32_t)v.w);
          if ((lane & 1) == 0) put_corr<kLds>(out, off / 32, -8 * t);
          if ((exports & kExpX8) && P.x8_out) *(int4 *)(P.x8_out + off) = v;
        }
      }
    }
    if ((exports & kExpX8) && P.e_x_out && pw == 0 && lane == 0) *P.e_x_out = P.e_x_given;
    return P.e_x_given;
  }
  if constexpr (NC == kPC) if (kDep && pro == PRO_EMUL_DYNQ8) {
    // ALU EMUL32 at p0 = 12 (gen_layer_script.py:1414-1418): clip16 of the
    // rounded product, then DYNQ8 below.  The second factor of the first
    // half of the chunks came with the inputs; the second half's is loaded
    // into the same registers once those are used.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1) pro_issue_x2(X, P, 1, pw, lane);
#pragma unroll
      for (int i = 0; i < kPC2; ++i) {
        const int c = h * kPC2 + i;
        if ((c * NP + pw) * kChunk < K) {
          const int4 a = X.x2[2 * i], b = X.x2[2 * i + 1];
          const int32_t av[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int64_t v = rshr64((int64_t)av[j] * piece_get(X.pc[c], j), kEmulP0);
            piece_set(X.pc[c], j, (int16_t)clamp64(v, -32768, 32767));
          }
        }
      }
    }
  }
  if (pro == PRO_RMSNORM_DYNQ8) {
    // layer_fixed.py:1262-1278 in sign-magnitude form (rshift_round rounds
    // the magnitude); K <= kStreamNormKMax
    // sum of squares: a pair's a^2 + b^2 <= 2^31 is exact as a uint32
    uint64_t ss = 0;
#pragma unroll
    for (int c = 0; c < kRN; ++c)
      if (kAll || (c * NP + pw) * kChunk < K) {
        const int32_t wd[4] = {X.pc[c].x, X.pc[c].y, X.pc[c].z, X.pc[c].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const s16x2 v = __builtin_bit_cast(s16x2, wd[j]);
          ss += (uint32_t)__builtin_amdgcn_sdot2(v, v, 0, false);
        }
      }
    ss = wave_sum_u64(ss);
    if (lane == 0) L.pss[pw] = (int64_t)ss;
    psync<NP>(L, ps, pw, lane, lspin);
    ss = 0;
#pragma unroll
    for (int w = 0; w < NP; ++w) ss += (uint64_t)L.pss[w];
    if (ss == 0) ss = 1;
    int64_t r;
    int e;
    rsqrt_q(ss, 2 * P.in_f + (31 - __clz(K)), L.rsqrt, &r, &e);
    const int s1 = 30 - e;
    const int32_t one = P.one_plus ? (1 << 14) : 0;
    // In double precision, exactly (doubles hold integers below 2^53, and
    // these operations round nothing below that):
    //   m = |x| * r < 2^15 * 2^31; rshift_round of a magnitude by s > 0 is
    //   floor(m * 2^-s + 1/2) (m * 2^-s + 1/2 < 2^52 has no bits below
    //   2^-s), a shift by s <= 0 is m * 2^-s, which may round above 2^53 --
    //   but y is then clipped to 2^32 - 1 (rounding keeps it >= 2^32), and
    //   below 2^32 it is exact (in_f within 0..40 is checked on the host, so
    //   the left shift is at most 17);
    //   q = (y * |w + one| + 8192) >> 14 = floor(y * |w + one| * 2^-14 + 1/2),
    //   y * |w + one| < 2^32 * 2^16.
    // A magnitude of 2^32 or more saturates the int16 result for any nonzero
    // scale exactly as 2^32 - 1 does, hence the clip of y.
    const double dr = (double)(uint32_t)r;
    const double dscale = s1 >= 0 ? __builtin_ldexp(1.0, -min(s1, 63))
                                  : __builtin_ldexp(1.0, min(-s1, 63));
    const double dhalf = s1 > 0 ? 0.5 : 0.0;
    const double drs = dr * dscale;   // exact: a power-of-2 scaling
#pragma unroll
    for (int c = 0; c < kRN; ++c) {
      const int base = (c * NP + pw) * kChunk + lane * 8;
      if (kAll || (c * NP + pw) * kChunk < K) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int32_t xv = piece_get(X.pc[c], j);
          const int32_t sc = (int32_t)piece_get(X.wv[c], j) + one;
          // |x| * r * 2^-s, rounded once, as fma(m, 2^-s, 1/2) of the exact m
          const double y = __builtin_fmin(
              __builtin_floor(__builtin_fma(__builtin_fabs((double)xv), drs, dhalf)), 4294967295.0);
          const double w14 = (double)abs(sc) * 0x1p-14;
          const double qd = __builtin_fmin(__builtin_floor(__builtin_fma(y, w14, 0.5)), 65535.0);
          const bool neg = (xv < 0) != (sc < 0);
          const int32_t qm = min((int32_t)qd, 32767 + (int32_t)neg);
          piece_set(X.pc[c], j, (int16_t)(neg ? -qm : qm));
        }
        if ((exports & kExpXn) && P.xn_out && base < K) *(int4 *)(P.xn_out + base) = X.pc[c];
      }
    }
  }
  u16x2 mx2 = (u16x2)(0);
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (kAll || (c * NP + pw) * kChunk < K) {
      mx2 = __builtin_elementwise_max(mx2, abs2(X.pc[c].x));
      mx2 = __builtin_elementwise_max(mx2, abs2(X.pc[c].y));
      mx2 = __builtin_elementwise_max(mx2, abs2(X.pc[c].z));
      mx2 = __builtin_elementwise_max(mx2, abs2(X.pc[c].w));
    }
  int32_t mx = max((int32_t)mx2.x, (int32_t)mx2.y);
  mx = wave_max_i32(mx);
  if (lane == 0) L.pmx[pw] = mx;
  psync<NP>(L, ps, pw, lane, lspin);
  mx = 0;
#pragma unroll
  for (int w = 0; w < NP; ++w) mx = max(mx, L.pmx[w]);
  // fixedpoint.py:24-33: the least e with rshift_round(max, e) <= 127 is
  // bitlen(max) - 7, or one more when rounding carries past 127
  int e = mx > 127 ? 25 - __clz(mx) : 0;
  if (e > 0 && ((mx + (1 << (e - 1))) >> e) > 127) ++e;
  const u16x2 half2 = (u16x2)((unsigned short)((1 << e) >> 1));
  const u16x2 e2 = (u16x2)((unsigned short)e);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int base = (c * NP + pw) * kChunk + lane * 8;
    if (kAll || (c * NP + pw) * kChunk < K) {
      const uint32_t lo = pack4(dynq2(X.pc[c].x, half2, e2), dynq2(X.pc[c].y, half2, e2));
      const uint32_t hi = pack4(dynq2(X.pc[c].z, half2, e2), dynq2(X.pc[c].w, half2, e2));
      // -8 * sum of the x8 met by the offset-form low nibbles of one
      // (group, quarter): 32 consecutive elements = the 4 lanes of a DPP quad
      int t4 = __builtin_amdgcn_sdot4((int)lo, 0x01010101, 0, false);
      t4 += __builtin_amdgcn_update_dpp(0, t4, 0xB1, 0xF, 0xF, false);
      t4 += __builtin_amdgcn_update_dpp(0, t4, 0x4E, 0xF, 0xF, false);
      if (kAll) {
        // (chunks past K write zeros into the buffer's unused room)
        put_x8<kLds>(out, base, lo, hi);
        if ((lane & 3) == 0) put_corr<kLds>(out, base / 32, -8 * t4);
      } else if (base < K) {
        put_x8<kLds>(out, base, lo, hi);
        if ((lane & 3) == 0) put_corr<kLds>(out, base / 32, -8 * t4);
        if ((exports & kExpX8) && P.x8_out) *(uint2 *)(P.x8_out + base) = make_uint2(lo, hi);
      }
    }
  }
  if ((exports & kExpX8) && P.e_x_out && pw == 0 && lane == 0) *P.e_x_out = e;
  return e;
}

// A stamped site's prologue for K <= 4608 (every site but the down
// projections), into LDS buffer b: code for three chunks per wavefront, not
// eight -- the prologue is a single wavefront's instruction stream, and the
// eight-chunk code spends most of its instructions on chunks past K (chained
// step 1.300 -> 1.272 ms, FFN blocks in layer order 0.623 -> 0.620 ms).  A
// function of its own: inlined, it changed the register allocation of the
// rest of the kernel (the FFN blocks interleaved 0.460 -> 0.494 ms, though
// that plan never runs it; 0.467 ms as it is).  The eight-chunk variant
// stays inlined: out of line it was slower everywhere (chained step 1.353
// ms).
struct SmallPro {
  int e;
  PSync ps;
  bool ok;
};
template <bool kDep, int NC = kPS, int NP = kPW>
__device__ __noinline__ SmallPro small_prologue(const GemvParams *Parg, int K, int pro,
                                                uint32_t stamp, int b, int exports, int pw,
                                                PSync ps, int32_t *err, uint32_t gspin,
                                                uint32_t lspin, int s) {
  CSite &P = *(CSite *)uniform_ptr(Parg);
  K = __builtin_amdgcn_readfirstlane(K);
  pro = __builtin_amdgcn_readfirstlane(pro);
  stamp = __builtin_amdgcn_readfirstlane(stamp);
  b = __builtin_amdgcn_readfirstlane(b);
  exports = __builtin_amdgcn_readfirstlane(exports);
  pw = __builtin_amdgcn_readfirstlane(pw);
  err = (int32_t *)uniform_ptr(err);
  s = __builtin_amdgcn_readfirstlane(s);
  Lds &L = g_lds;
  const int lane = lane_now();
  ProXN<NC> X;
  SmallPro r;
  r.ok = pro_issue_stamped<NC, NP>(X, P, K, pro, stamp, pw, lane, err, gspin);
  if (NP == kPW) {
    r.e = group_prologue<true, kDep, NC, NP>(P, K, pro, L, L.x[b], exports, pw, lane, ps, X,
                                             lspin);
    r.ps = ps;
  } else {
    // with the control wavefront: barrier phases 2s + 1, 2s + 2 of site s
    PSync p4{2 * s, 1};
    r.e = group_prologue<true, kDep, NC, NP>(P, K, pro, L, L.x[b], exports, pw, lane, p4, X,
                                             lspin);
    r.ps = ps;
    r.ok = r.ok && p4.ok;
  }
  return r;
}

// The control wavefront computes a share of site s's prologue with the
// three prologue wavefronts (two chunks of 512 elements each of the four,
// for K <= 4096, instead of three chunks each of the three) when it is idle
// then: in a dependent plan, at a site whose stamped input is the site just
// before it, whose outputs this CU's control wavefront has then just stored
// (and whose other CUs' outputs the prologue waits for anyway).  Chained
// step 1.235 -> 1.202 ms, FFN blocks in layer order 0.617 -> 0.621 ms and
// interleaved 0.467 -> 0.471 ms (plans that never run it: the code moved);
// the weight wavefronts wait for the fourth flag at such sites only (the
// prologue wavefronts posting it at every other site cost the FFN blocks
// 0.617 -> 0.630 ms).
constexpr int kAssistKMax = 2 * kPR * kChunk;   // 4096
template <bool kDep>
__device__ __forceinline__ bool ctrl_assists(CSite &P, int s) {
  return kDep && P.local_pro && P.stamp_src >= 0 && P.stamp_src == s - 1 && P.K <= kAssistKMax;
}

// Site s's prologue, by the CU that owns it: inputs, compute, then -- every
// store of the three wavefronts complete -- e_x and the site's flag.
template <bool kDep>
__device__ PSync compute_publish(CSite &P, Lds &L, int8_t *stg, uint32_t *flag, uint32_t epoch,
                                 int pw, int lane, PSync ps, uint32_t lspin) {
  ProX X;
  pro_issue<kDep>(X, P, pw, lane);
  const int e =
      group_prologue<false, kDep>(P, P.K, P.pro, L, stg, kExpX8 | kExpXn, pw, lane, ps, X, lspin);
  if (pw == 0 && lane == 0) store_coherent((int32_t *)(stg + kXB), (int32_t)e);
  wait_vm_all();
  psync(L, ps, pw, lane, lspin);
  if (pw == 0 && lane == 0) store_coherent(flag, epoch);
  return ps;
}

// A site whose prologue every CU computes itself (local) has its x8 and e_x
// exported by CU s % G's control wavefront, from the site's LDS buffer, and
// not by its prologue wavefronts: their stores would count in the same
// in-order counter as their polls for the next site's input, which then
// waited for the stores to complete, and that CU became the slowest at
// every site (chained step 1.402 -> 1.371 ms).  The buffer is not reused
// before the export is done (L.xdone).
__device__ __forceinline__ bool ctrl_exports(CSite &P, int s, int r, int G) {
  return P.local_pro && site_owner(s, G) == r && (P.x8_out != nullptr || P.e_x_out != nullptr);
}
template <bool kDep>
__device__ __forceinline__ void wait_exported(CSite *sites, Lds &L, int t, int r, int G, int lane,
                                              uint32_t lspin, bool &ok) {
  if (kDep && t >= 0 && ctrl_exports(sites[t], t, r, G)) ok = lds_wait_ge(&L.xdone, t, lspin) && ok;
}

// The wavefront waits until the first `need` of sites s .. s + n - 1 (flags
// flag[0 .. n), need <= n <= 64) have their activations staged in this
// launch, and returns how many of the n, from the first, are (bounded; on
// giving up it returns fewer than need, with bit 1 of err, as for the
// grid-wide wait).
constexpr int kStageBatch = 4;   // staged sites copied per round trip, at most ...
constexpr int kStageBlocks = 2 * kCW;   // ... with this many weight blocks per CU in all
static_assert(kStageBatch < kNB, "a batch's buffers are free together");
// a site's weight blocks on one CU, at most
__device__ __forceinline__ int site_blocks(CSite &P, int G) {
  return (P.tiles_q + (P.tiles_r > 0 ? 1 : 0)) * P.nblk;
}
__device__ __forceinline__ int wait_staged_n(const uint32_t *flag, int n, int need,
                                             uint32_t epoch, int lane, int32_t *err,
                                             uint32_t gspin) {
  for (uint32_t it = 0; it < gspin; ++it) {
    const bool mine = lane < n && __hip_atomic_load(flag + lane, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT) >= epoch;
    // sites from the first on that are staged: the lowest lane that is not
    const uint64_t notyet = ~__ballot(mine);
    const int run = notyet ? __builtin_ctzll(notyet) : 64;
    if (run >= need) return run < n ? run : n;
    __builtin_amdgcn_s_sleep(1);
  }
  if (lane == 0) atomicOr(err, 2);
  return 0;
}

// copy a staged site (x8 [0, K), corrections [kXloOff, + K/8)) into LDS
// buffer xb: 1 KiB per copy instruction, split over the 3 wavefronts
__device__ __forceinline__ void load_staged(const int8_t *stg, int8_t *xb, int K, int pw,
                                            int lane) {
  for (int off = pw * 1024; off < K; off += kPW * 1024)
    if (off + 16 * lane < K) copy16_sc1(stg + off + 16 * lane, lds_off(xb + off));
  const int nlo = K / 8;
  for (int off = pw * 1024; off < nlo; off += kPW * 1024)
    if (off + 16 * lane < nlo)
      copy16_sc1(stg + kXloOff + off + 16 * lane, lds_off(xb + kXloOff + off));
}

// the wavefront waits until all prologue wavefronts have written site s's
// activations into buffer b (bounded, like lds_wait_eq).  Polled at a long
// interval (about 1,000 cycles): eight weight wavefronts waiting here share
// their SIMDs with the prologue wavefronts that compute the activations, and
// polling every 64 cycles slowed those (the chained step by 4 %, the
// independent one by 2 %); 2,000 cycles was slower again on the chained step.
// (with_ctrl: the control wavefront has a share of the site's prologue, and
// its flag counts too)
__device__ __forceinline__ void wait_ready(Lds &L, int b, int s, int lane, uint32_t lspin,
                                           bool with_ctrl) {
  const int f = with_ctrl ? (lane & (kPR - 1)) : lane % kPW;
  for (uint32_t n = 0;; ++n) {
    if (__all(lds_read_i32(&L.ready[b][f]) == s)) break;
    if (lds_read_i32(&L.abort) != 0) break;
    if (n > lspin) {
      if (lane == 0) {
        lds_write_i32(&L.abort, 1);
        lds_or_i32(&L.err, 4);
      }
      break;
    }
    __builtin_amdgcn_s_sleep(16);
  }
  wait_lds();
}

// the wavefront waits until every weight wavefront has moved past site t
__device__ __forceinline__ bool wait_weights_past(Lds &L, int t, int lane, uint32_t lspin) {
  for (uint32_t n = 0; n < lspin; ++n) {
    if (__all(lds_read_i32(&L.wsite[lane & (kCW - 1)]) > t)) return true;
    if (lds_read_i32(&L.abort) != 0) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}


// The head's maximum over workgroups: each adds its key with an atomic max,
// waits for it to be performed, then counts itself in; the last to arrive
// reads the key, writes (index, value) and zeroes both words for the next
// launch, which the stream orders after this one.  The atomics are performed
// at the device's coherence point, so, as for the completion flags, a wait
// for the returned value orders them -- an acquire / release pair would add
// an L2 write-back and invalidate to every workgroup's exit.
// A key is (value ^ 2^31) << 32 | (2^32 - 1 - index): the unsigned maximum is
// the largest value and, among equal values, the lowest index.
__device__ __forceinline__ void head_arrive(const StreamParams &S, int G, uint64_t best) {
  const size_t w0 = stream_head_word0(G, S.nsites);
  uint64_t *key = (uint64_t *)(S.done + w0);
  uint32_t *count = S.done + w0 + 2;
  uint64_t was = __hip_atomic_fetch_max(key, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" : "+v"(was));   // a returning atomic ...
  wait_vm_all();                   // ... that has returned
  const uint32_t before =
      __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (before != (uint32_t)G - 1u) return;
  const uint64_t k = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(key, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  S.result[0] = (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu));
  S.result[1] = (int32_t)((uint32_t)(k >> 32) ^ 0x80000000u);
}

// The prologue wavefronts' program: every site's activations, in order,
// into the LDS ring.  Inlined into the kernel (the three-chunk stamped
// prologue excepted, see small_prologue); the arguments are made
// wavefront-uniform, so table reads stay scalar.
template <bool kDep>
__device__ __forceinline__ void prologue_role(const GemvParams *sites_arg, int nsites, int r,
                                           int G, int wave, uint32_t *done, int8_t *stage,
                                           uint32_t epoch, int32_t *err, uint32_t gspin,
                                           uint32_t lspin) {
  Lds &L = g_lds;
  CSite *sites = (CSite *)uniform_ptr(sites_arg);
  done = (uint32_t *)uniform_ptr(done);
  stage = (int8_t *)uniform_ptr(stage);
  err = (int32_t *)uniform_ptr(err);
  nsites = __builtin_amdgcn_readfirstlane(nsites);
  r = __builtin_amdgcn_readfirstlane(r);
  G = __builtin_amdgcn_readfirstlane(G);
  wave = __builtin_amdgcn_readfirstlane(wave);
  epoch = __builtin_amdgcn_readfirstlane(epoch);
  const uint32_t fbase = (epoch - 1u) * (uint32_t)(nsites + 1);
  const int lane = lane_now();
  // Every site's prologue is computed once, by CU s % G, into the site's
  // staging area (a site behind no fence at once, a fenced one after its
  // grid-wide wait); every CU then copies the staged sites, in order, into
  // its buffer ring ahead of the weight wavefronts.
  const int pw = wave - kPW0;
  // (default wave priority: these wavefronts mostly wait, and raised
  // priority lets their polls outrank the weight wavefronts' work)
  PSync ps{0, 1};
  uint32_t *sflag = done + stream_flag_site0(G);
  bool ok = true;
  // (a site whose prologue every CU computes itself -- one reading stamped
  // words has no fence yet depends on its producer -- is not staged: its
  // inputs are not written yet)
  for (int s = r; s < nsites; s += G)
    if (sites[s].fence_at == 0 && !(kDep && sites[s].local_pro))
      ps = compute_publish<kDep>(sites[s], L, stage + (size_t)s * kStageBytes, sflag + s, epoch,
                           pw, lane, ps, lspin);
  for (int s = 0; s < nsites; ++s) {
    // lane-derived addresses are recomputed per site, so the compiler does
    // not keep them live
    const int lane = lane_now();
    CSite &P = sites[s];
    const int8_t *stg = stage + (size_t)s * kStageBytes;
    const int b = s % kNB;
    if (kDep) touch_site(&P);
    if (kDep && P.local_pro) {
      // behind a fence, every CU computes the site's prologue itself,
      // straight into its LDS buffer: one read of the inputs after the
      // grid-wide wait, instead of a staged copy that would first have to
      // be computed, published and flagged by one CU
      if (s >= kNB) ok = wait_weights_past(L, s - kNB, lane, lspin) && ok;
      wait_exported<kDep>(sites, L, s - kNB, r, G, lane, lspin, ok);
      ok = lds_wait_ge(&L.gridok, P.fence_at, lspin) && ok;
      // the fields the prologue branches on, read before its waits
      int pK = P.K, ppro = P.pro;
      const int exports = site_owner(s, G) == r ? kExpXn : 0;
      int e;
      if (P.stamp_src >= 0) {
        // no grid-wide wait: the input's own words say when it is whole.
        // Polled once this CU has stored its own share (a CU that polls
        // while others still stream would only add traffic).
        ok = lds_wait_ge(&L.served, P.stamp_src, lspin) && ok;
      }
      const bool assisted = ctrl_assists<kDep>(P, s);
      if (P.stamp_src >= 0 && pK <= kStampKSmall) {
        const uint32_t stamp = fbase + (uint32_t)P.stamp_src + 1u;
        const SmallPro sp =
            assisted ? small_prologue<kDep, 2, kPR>(sites_arg + s, pK, ppro, stamp, b, exports,
                                                    pw, ps, err, gspin, lspin, s)
                     : small_prologue<kDep>(sites_arg + s, pK, ppro, stamp, b, exports, pw, ps,
                                            err, gspin, lspin, s);
        e = sp.e;
        ps = sp.ps;
        ok = sp.ok && ok;
      } else {
        ProX X;
        if (P.stamp_src >= 0)
          ok = pro_issue_stamped(X, P, pK, ppro, fbase + (uint32_t)P.stamp_src + 1u, pw, lane,
                                 err, gspin) &&
               ok;
        else
          pro_issue<kDep>(X, P, pw, lane);
        // held in registers across the waits: read again after them, the
        // fields' scalar loads could miss
        asm volatile("" : "+s"(pK), "+s"(ppro));
        e = group_prologue<true, kDep>(P, pK, ppro, L, L.x[b], exports, pw, lane, ps, X, lspin);
      }
      if (lane == 0) {
        if (pw == 0) lds_write_i32(&L.ex[b], e);
        lds_write_i32(&L.ready[b][pw], s);
      }
      continue;
    }
    if (site_owner(s, G) == r && P.fence_at > 0) {
      ok = lds_wait_ge(&L.gridok, P.fence_at, lspin) && ok;
      ps = compute_publish<kDep>(P, L, stage + (size_t)s * kStageBytes, sflag + s, epoch, pw,
                           lane, ps, lspin);
    }
    // Staged sites go in batches: the consecutive sites s .. e - 1 that wait
    // for no other workgroup (their staging flags went up at launch start)
    // are polled in one round trip, copied, and waited for once.  One site
    // at a time, every site cost two dependent round trips behind the weight
    // stream, about 2.5 us, which bounded runs of small sites.
    // (only small sites go together: while the batch's blocks on this CU fit
    // the weight wavefronts' registers; a large site's readiness would
    // otherwise wait for the copies of the sites after it)
    int e = s + 1;
    if (P.fence_at == 0) {
      int blocks = site_blocks(P, G);
      while (e < nsites && e < s + kStageBatch && sites[e].fence_at == 0 &&
             !(kDep && sites[e].local_pro) && blocks + site_blocks(sites[e], G) <= kStageBlocks) {
        blocks += site_blocks(sites[e], G);
        ++e;
      }
    }
    if (e - 1 >= kNB) ok = wait_weights_past(L, e - 1 - kNB, lane, lspin) && ok;
    for (int t = s; kDep && t < e; ++t) wait_exported<kDep>(sites, L, t - kNB, r, G, lane, lspin, ok);
    ok = wait_staged_n(sflag + s, e - s, e - s, epoch, lane, err, gspin) >= e - s && ok;
    for (int t = s; t < e; ++t)
      load_staged(stage + (size_t)t * kStageBytes, L.x[t % kNB], sites[t].K, pw, lane);
    // lane j: e_x of site s + j
    const int exj = lane < e - s ? __hip_atomic_load((const int32_t *)(stg + (size_t)lane *
                                                                        kStageBytes + kXB),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                 : 0;
    wait_vm_all();
    // this wavefront's copies into the batch's buffers have landed
    // (lds_write_i32 waits for its LDS work first); a site is ready once all
    // three have posted
    for (int t = s; t < e; ++t) {
      const int ex = __builtin_amdgcn_readlane(exj, t - s);
      if (lane == 0) {
        if (pw == 0) lds_write_i32(&L.ex[t % kNB], ex);
        lds_write_i32(&L.ready[t % kNB][pw], t);
      }
    }
    s = e - 1;
  }
  if (!(ok && ps.ok) && lane_now() == 0) lds_or_i32(&L.err, 4);
}

// The TOPK-32 head's scan, by prologue wavefront 0 of workgroup r once the
// plan's last prologue is done: chunks c = r, r + G, ... of the scan of
// w4a8_topk_device.h, each as soon as its rows' stamped words all carry
// this launch's stamp -- while the head still streams its later tiles.  A
// chunk's rows are stored by other workgroups' control wavefronts, which
// never wait for a prologue wavefront once the head's activations are
// ready; a chunk waits only for the lists of lower-numbered chunks, so
// every wait ends as long as every workgroup is resident (bounded: err bit
// 3).  Only in the kernel instances for plans with a TOPK-32 head.
__device__ __forceinline__ void topk_role(const uint64_t *ys, uint64_t *lists, int32_t *flags,
                                       int32_t *out, int32_t n, uint32_t stamp, uint32_t epoch,
                                       int32_t *err, uint32_t spin, int r, int G) {
  Lds &L = g_lds;
  ys = (const uint64_t *)uniform_ptr(ys);
  lists = (uint64_t *)uniform_ptr(lists);
  flags = (int32_t *)uniform_ptr(flags);
  out = (int32_t *)uniform_ptr(out);
  err = (int32_t *)uniform_ptr(err);
  n = __builtin_amdgcn_readfirstlane(n);
  stamp = __builtin_amdgcn_readfirstlane(stamp);
  epoch = __builtin_amdgcn_readfirstlane(epoch);
  spin = __builtin_amdgcn_readfirstlane(spin);
  r = __builtin_amdgcn_readfirstlane(r);
  G = __builtin_amdgcn_readfirstlane(G);
  const int lane = threadIdx.x & 63;
  const bool up = tk::tk_ror4_up();
  const int nchunks = n <= tk::kTkFirst ? 1 : 1 + (n - tk::kTkFirst + tk::kTkRows - 1) / tk::kTkRows;
  uint64_t *part = lists, *sup = lists + (size_t)nchunks * tk::kTk;
  bool ok = true;
  for (int c = r; c < nchunks; c += G) {
    const int64_t s0 = tk::chunk_first(c), end = tk::chunk_end(c, n);
    // the chunk's words through a buffer whose range ends with them: lanes
    // past the end read zero and count as arrived
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(ys + s0), (short)0, (int)((end - s0) * 8), kBufDword3);
    int32_t yv[tk::kTkPerLane];
    // First a light poll, one word per tile (lane l: the first row of the
    // chunk's tile l; a tile's rows are stored by one instruction), so that
    // the wait for a chunk whose rows come late -- the last chunks wait for
    // most of the head -- takes 512 bytes a poll instead of 8 KB from the
    // weight stream's bandwidth.
    bool all = false;
    for (uint32_t it = 0; it < spin && !all; ++it) {
      if (it > 0) __builtin_amdgcn_s_sleep(8);
      typedef uint32_t u2 __attribute__((ext_vector_type(2)));
      const u2 w = __builtin_amdgcn_raw_buffer_load_b64(rs, lane * kTileRows * 8, 0, kAuxSc1);
      all = __all(s0 + lane * kTileRows >= end || w.y == stamp);
    }
    all = false;
    for (uint32_t it = 0; it < spin && !all; ++it) {
      if (it > 0) __builtin_amdgcn_s_sleep(2);
      bool mine = true;
#pragma unroll
      for (int t = 0; t < tk::kTkPerLane; ++t) {
        const int i = lane + 64 * t;
        typedef uint32_t u2 __attribute__((ext_vector_type(2)));
        const u2 w = __builtin_amdgcn_raw_buffer_load_b64(rs, i * 8, 0, kAuxSc1);
        yv[t] = (int32_t)w.x;
        mine = mine && (s0 + i >= end || w.y == stamp);
      }
      all = __all(mine);
    }
    ok = ok && all;
    ok = tk::chunk_run(yv, L.tkrows, L.tkbuf, n, nchunks, c, (int32_t)epoch, part, sup, flags,
                       out, spin, up, lane) && ok;
  }
  if (!ok && lane == 0) atomicOr(err, 8);
}

// The weight wavefronts' program.  (As a function of its own, with a
// register allocation apart from the other roles', it ran 1-2 % slower on
// the independent-input stream and 2.5 % slower on the chained one than
// inlined, so it is inlined.)  The arguments are made wavefront-uniform, so
// table reads stay scalar loads.
template <bool kDep>
__device__ __forceinline__ void weight_role(const GemvParams *sites_arg, int nsites, int r,
                                            int G, int wave, uint32_t lspin) {
  Lds &L = g_lds;
  CSite *sites = (CSite *)uniform_ptr(sites_arg);
  nsites = __builtin_amdgcn_readfirstlane(nsites);
  r = __builtin_amdgcn_readfirstlane(r);
  G = __builtin_amdgcn_readfirstlane(G);
  wave = __builtin_amdgcn_readfirstlane(wave);
  const int tid = threadIdx.x, lane = tid & 63;
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
  // consume the block in R (item c; this wavefront's next item is nx),
  // refill R with the item two ahead, and add into the tile after this
  // wavefront's last block of it
  auto step = [&](BlockRegs &R, Cursor &c, const Cursor &nx) {
    // the lane-derived addresses are recomputed per step, so the compiler
    // does not keep them all live
    const int lane_s = lane_now();
    if (c.s != s_cur) {
      // done with every earlier site; wait for this one's activations
      s_cur = c.s;
      lds_write_i32(&L.wsite[wave], s_cur);
      wait_ready(L, s_cur % kNB, s_cur, lane_s, lspin, ctrl_assists<kDep>(sites[s_cur], s_cur));
      e_x = __builtin_amdgcn_readfirstlane(lds_read_i32(&L.ex[s_cur % kNB]));
      contributors = min(c.nblk, kCW);
    }
    CSite &P = sites[c.s];
    const int i = c.i, b = c.b;
    const int8_t *xb = L.x[c.s % kNB];
    p = dot_block(R, groups_in(c.ng, b), b * kGroupsPerBlock, lane_s & 3, xb,
                  (const int32_t *)(xb + kXloOff), p);
    const bool last = !(nx.s == c.s && nx.i == i);
    const Cursor done = c;
    auto finish_tile = [&]() {
      const int kt = done.kt0 + i;
      if (tile_add(L, kt, p, contributors, lspin, lane_s)) {
        const int t = done.first + i * G;
        tile_epilogue(L, kt, done.jepi, done.jrows, t - done.jtile0, e_x, lane_s);
      }
      p = 0;
    };
    // In the instances for plans with waits, a tile is finished before the
    // refill: the refill's cursor reads table entries of sites further
    // ahead, and its nine loads queue behind the other wavefronts' refills,
    // and both would delay the tile's completion -- which a site waiting
    // for this one's outputs needs (chained step 1.418 -> 1.401 ms, the FFN
    // blocks in layer order 0.682 -> 0.650 ms; with each down projection
    // after the next gate / up, where nothing waits, 0.498 -> 0.512 ms).
    // Otherwise the refill goes first, to keep the weight stream full.
    const bool finish_first = kDep;
    if (last && finish_first) finish_tile();
    c = cn;
    cur_next(sites, nsites, r, G, cn);
    issue_block(R, sites, nsites, G, c, lane_s);
    if (last && !finish_first) finish_tile();
  };
  for (;;) {
    if (ca.s >= nsites) break;
    step(A, ca, cb);
    if (cb.s >= nsites) break;
    step(B, cb, ca);
  }
  lds_write_i32(&L.wsite[wave], nsites);
}

// kSpin: the context set its own spin limits (a test of the give-up paths);
// otherwise the limits are the compile-time defaults, which the waits fold
// in (runtime limits everywhere cost 1 % on the independent-input stream and
// 5 % on the chained one).  kTopk: the plan ends in a TOPK-32 head (the scan
// code stays out of the other instances)
template <bool kDep, bool kSpin, bool kTopk>
__global__ __launch_bounds__(kThreads) void stream_kernel(StreamParams S,
                                                          const GemvParams *__restrict__ sites_arg) {
  CSite *sites = (CSite *)sites_arg;
  Lds &L = g_lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, r = blockIdx.x;
  const int nsites = S.nsites;
  // this launch's completion-flag values are fbase + 1 .. fbase + nsites
  const uint32_t fbase = (S.epoch - 1u) * (uint32_t)(nsites + 1);
  // polls before a wait gives up: between workgroups, within one
  const uint32_t gspin = kSpin && S.grid_spin ? S.grid_spin : kGridSpin;
  const uint32_t lspin = kSpin && S.lds_spin ? S.lds_spin : kLdsSpin;

  // tables, reduction slots and flags
  const int32_t *tab = sites[0].tables;
  for (int i = tid; i < 512; i += kThreads) L.rsqrt[i] = (uint16_t)tab[kRsqrtOff + i];
  for (int i = tid; i < 257; i += kThreads) L.sig[i] = (uint16_t)tab[kSigmoidOff + i];
  for (int i = tid; i < kTSlots * kTileRows; i += kThreads) (&L.tv[0][0])[i] = 0;
  if (tid < kTSlots) {
    L.tcnt[tid] = 0;
    L.tgen[tid] = tid;
    L.tready[tid] = 0;
  }
  if (tid < kNB * kPR) (&L.ready[0][0])[tid] = -1;
  if (tid < kCW) L.wsite[tid] = 0;
  if (tid < kPW) L.psync[tid] = 0;
  if (tid < kPR) L.psync4[tid] = 0;
  if (tid == 0) {
    L.served = -1;
    L.xdone = -1;
    L.gridok = 0;
    L.abort = 0;
    L.err = 0;
    L.best = 0;
  }
  wait_vm_all();   // the table loads, before any weight load is counted
  lds_barrier();

  if (wave == kCtrl) {
    // outputs of every site in order; at a fenced site, the grid-wide wait
    int kt0 = 0;   // CU-local number of the site's first tile
    for (int s = 0; s < nsites; ++s) {
      CSite &P = sites[s];
      if (S.trace && r == 0 && lane == 0) S.trace[s] = wall_clock64();
      // the next sites' table entries, for the waits, epilogues and weight
      // cursors around their fences
      if (kDep)
        for (int a = s + 1; a < nsites && a <= s + 3; ++a) touch_site(&sites[a]);
      ctrl_serve<kDep>(P, L, kt0, r, G, lane, fbase + (uint32_t)s + 1u, lspin);
      if (kDep && lane == 0) lds_write_i32(&L.served, s);
      if (kDep && ctrl_exports(P, s, r, G)) {
        // x8 and e_x from the site's LDS buffer, after the post that lets
        // this CU poll for the next site's input; once the site's prologue
        // is done here (a CU with no tile of the site has not waited for it)
        const int b = s % kNB;
        wait_ready(L, b, s, lane, lspin, ctrl_assists<kDep>(P, s));
        if (P.x8_out)
          for (int off = 16 * lane; off < P.K; off += 1024)
            *(int4 *)(P.x8_out + off) = *(const int4 *)(L.x[b] + off);
        if (P.e_x_out && lane == 0) *P.e_x_out = lds_read_i32(&L.ex[b]);
        if (lane == 0) lds_write_i32(&L.xdone, s);
      }
      kt0 += site_ntl(P, site_first(P, r, G));
      if (s + 1 < nsites && sites[s + 1].fence) {
        const uint32_t v = fbase + (uint32_t)(s + 1);
        wait_vm_all();   // this workgroup's outputs of sites <= s are stored
        if (lane == 0) store_coherent(S.done + r, v);
        grid_wait(S.done, G, v, lane, S.err, gspin);
        if (lane == 0) lds_write_i32(&L.gridok, s + 1);
      }
      if (s + 1 < nsites && ctrl_assists<kDep>(sites[s + 1], s + 1)) {
        // this wavefront's share of the next site's prologue (its input is
        // the site just stored); its buffer is free once every weight
        // wavefront has left the site that used it last (this wavefront's
        // own exports of that site are done)
        const int t = s + 1, b = t % kNB;
        CSite &Q = sites[t];
        bool aok = t < kNB || wait_weights_past(L, t - kNB, lane, lspin);
        const SmallPro sp = small_prologue<kDep, 2, kPR>(
            sites_arg + t, Q.K, Q.pro, fbase + (uint32_t)t, b, site_owner(t, G) == r ? kExpXn : 0,
            kPW, PSync{0, 1}, S.err, gspin, lspin, t);
        aok = aok && sp.ok;
        if (lane == 0) {
          lds_write_i32(&L.ready[b][kPW], t);
          if (!aok) lds_or_i32(&L.err, 4);
        }
      }
    }
  } else if (wave >= kPW0) {
    prologue_role<kDep>(sites_arg, S.nsites, r, G, wave, S.done, S.stage, S.epoch, S.err,
                        gspin, lspin);
    // the TOPK-32 head is the last site: its stamp is that of site nsites - 1
    if (kTopk && wave == kPW0)
      topk_role(S.topk_y, S.topk_lists, S.topk_flags, S.topk_out, S.topk_rows,
                fbase + (uint32_t)nsites, S.epoch, S.err, gspin, r, G);
  } else {
    weight_role<kDep>(sites_arg, nsites, r, G, wave, lspin);
  }

  const int lane_e = lane_now();
  lds_barrier();
  if (wave == kCtrl && lane_e == 0) {
    const int32_t e = lds_read_i32(&L.err);
    if (e) atomicOr(S.err, e);
    if (S.head_site >= 0) head_arrive(S, G, L.best);
    if (S.trace && r == 0) S.trace[nsites] = wall_clock64();
  }
}

}  // namespace

hipError_t launch_stream(const StreamParams &sp, int grid, hipStream_t s, bool cooperative,
                         bool dependent, hipEvent_t start, hipEvent_t stop) {
  const GemvParams *sites = sp.sites;
  const bool spin = sp.grid_spin || sp.lds_spin;
  auto kernel =
      sp.topk_out
          ? (dependent ? (spin ? stream_kernel<true, true, true> : stream_kernel<true, false, true>)
                       : (spin ? stream_kernel<false, true, true>
                               : stream_kernel<false, false, true>))
          : (dependent ? (spin ? stream_kernel<true, true, false>
                               : stream_kernel<true, false, false>)
                       : (spin ? stream_kernel<false, true, false>
                               : stream_kernel<false, false, false>));
  if (cooperative) {
    void *args[] = {(void *)&sp, (void *)&sites};
    hipError_t e = start ? hipEventRecord(start, s) : hipSuccess;
    if (e == hipSuccess)
      e = hipLaunchCooperativeKernel((const void *)kernel, dim3(grid), dim3(kThreads), args, 0,
                                     s);
    if (e == hipSuccess && stop) e = hipEventRecord(stop, s);
    return e;
  }
  // events, when given, are recorded by the dispatch itself
  hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, s, start, stop, 0, sp, sites);
  return hipGetLastError();
}

int stream_max_blocks_per_cu() {
  int n = 1 << 30;
  for (auto k : {stream_kernel<false, false, false>, stream_kernel<true, false, false>,
                 stream_kernel<false, true, false>, stream_kernel<true, true, false>,
                 stream_kernel<false, false, true>, stream_kernel<true, false, true>,
                 stream_kernel<false, true, true>, stream_kernel<true, true, true>}) {
    int m = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&m, k, kThreads, 0) != hipSuccess) return 1;
    n = m < n ? m : n;
  }
  return n < 1 ? 1 : (n > 1 ? 1 : n);
}

size_t stream_counter_words(int grid, int nsites) {
  return stream_head_word0(grid, nsites) + 64;
}

}  // namespace w4a8
