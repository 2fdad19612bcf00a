// TOPK-32 device routines shared by the stand-alone TOPK kernel
// (w4a8_topk.hip) and the persistent plan's LM head (w4a8_stream.hip): the
// layer_topk32 block of docs/SEQ_ISA.md B8 (the model of
// tb/scripts/gen_topk_cases.py:60-104) -- the 32 largest head values,
// sorted by value descending with ties in arrival order (the lower row
// first), a count saturating at 32, and the sticky overflow bit, set when an
// arrival is rejected (the list full and the arrival not greater than
// entry[31]) while exactly equal to entry[31].
//
// A row's key is (value ^ 2^31) << 32 | (2^32 - 1 - row): key order is
// (value desc, row asc), so the list is the 32 largest keys of the whole
// head -- the same for any split of the rows, so it is found chunk by chunk
// in parallel.  The overflow bit depends on the arrival order, so each chunk
// (1024 rows; the first 256) replays its own arrivals against the list of
// everything before it (built from the earlier chunks' lists); only arrivals
// at or above the running entry[31] can insert or tie, and since entry[31]
// only rises, an arrival below it when its 64-row group starts stays below.
//
// One wavefront per chunk.  A chunk publishes its own list; the last chunk
// of each run of 16 (a super-chunk) also publishes the run's list.  The list
// before chunk c is then the merge of at most 15 super lists and 15 chunk
// lists.  A chunk only waits for lower-numbered chunks, each of which
// publishes before it waits, so the waits end as long as every chunk's
// wavefront runs; the last chunk gathers the result.  Flags carry an epoch,
// so they are never cleared between uses; data crossing workgroups moves
// with agent-coherent accesses.
#pragma once
#include "w4a8_internal.h"

namespace w4a8 {
namespace tk {
namespace {

constexpr int kTkRows = 1024;   // rows per chunk, but the first
constexpr int kTkFirst = 256;   // rows of chunk 0: its replay starts from an
                                // empty list, so it is kept short
constexpr int kTk = 32;
constexpr int kTkPerLane = kTkRows / 64;
constexpr int kTkSerialMax = 12;   // candidates a group replays one by one

__device__ __forceinline__ uint64_t tk_key(int32_t v, uint32_t row) {
  return ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | (uint64_t)(0xFFFFFFFFu - row);
}
__device__ __forceinline__ int32_t tk_val(uint64_t k) {
  return (int32_t)((uint32_t)(k >> 32) ^ 0x80000000u);
}
__device__ __forceinline__ uint32_t tk_row(uint64_t k) {
  return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu);
}
// lane - 1's value (DPP wave_shr:1; lane 0 keeps its own)
__device__ __forceinline__ uint64_t shift_up1_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)v, (int)(uint32_t)v,
                                                            0x138, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(v >> 32),
                                                            (int)(uint32_t)(v >> 32), 0x138, 0xF,
                                                            0xF, false);
  return ((uint64_t)hi << 32) | lo;
}
// lane j's 64-bit value (j uniform)
__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int j) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, j);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), j);
  return ((uint64_t)hi << 32) | lo;
}

// Lane exchange x[lane ^ m], without LDS.  Distances 1 and 2 are DPP quad
// permutes, 8 is a DPP rotation by 8 within a row of 16 lanes (its own
// inverse), 4 takes the rotations by 4 and by 12 (one brings lane + 4, the
// other lane - 4; `ror4_up` says which, found once per wavefront by
// tk_ror4_up), 16 and 32 are the gfx950 row swaps v_permlane16_swap (odd
// rows of 16 with even rows) and v_permlane32_swap (halves).
__device__ __forceinline__ bool tk_ror4_up() {
  const int t = __builtin_amdgcn_update_dpp(0, (int)(threadIdx.x & 63), 0x124, 0xF, 0xF, false);
  return __builtin_amdgcn_readfirstlane(t) == 4;   // lane 0 read lane 4
}
__device__ __forceinline__ uint32_t xchg32(uint32_t x, int m, bool ror4_up, int lane) {
  switch (m) {
    case 1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);
    case 2: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
    case 4: {
      const uint32_t a = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x124, 0xF, 0xF, false);
      const uint32_t b = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x12C, 0xF, 0xF, false);
      const bool want_up = (lane & 4) == 0;   // lanes with bit 2 clear read lane + 4
      return want_up == ror4_up ? a : b;
    }
    case 8: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);
    case 16: {
      // {x with odd rows <- even rows, x with even rows <- odd rows}
      const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
      return (lane & 16) ? r[0] : r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
      return (lane & 32) ? r[0] : r[1];
    }
  }
}
__device__ __forceinline__ uint64_t xchg64(uint64_t v, int m, bool ror4_up, int lane) {
  const uint32_t lo = xchg32((uint32_t)v, m, ror4_up, lane);
  const uint32_t hi = xchg32((uint32_t)(v >> 32), m, ror4_up, lane);
  return ((uint64_t)hi << 32) | lo;
}

// bitonic sort of the wavefront's 64 keys, descending across the lanes
__device__ __forceinline__ uint64_t sort64(uint64_t v, bool ror4_up, int lane) {
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t o = xchg64(v, stride, ror4_up, lane);
      const bool desc = size == 64 || (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      v = lower == desc ? (v > o ? v : o) : (v < o ? v : o);
    }
  }
  return v;
}

// One bitonic merge: lanes 0..31 descending and 32..63 ascending (a bitonic
// sequence) become 64 keys descending, the top 32 in lanes 0..31.
__device__ __forceinline__ uint64_t bmerge64(uint64_t v, bool ror4_up, int lane) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    const uint64_t o = xchg64(v, s, ror4_up, lane);
    v = (lane & s) == 0 ? (v > o ? v : o) : (v < o ? v : o);
  }
  return v;
}

// Lanes 0..31 of L and of V each hold 32 keys sorted descending; afterwards
// lanes 0..31 hold the top 32 of both, descending (lanes 32..63: unspecified).
// max(L[i], V[31 - i]) holds the top 32 as a bitonic sequence; five
// half-cleaner stages sort it.  V[31 - i] = row_mirror, then the row swap.
__device__ __forceinline__ uint64_t merge32v(uint64_t L, uint64_t V, bool ror4_up, int lane) {
  const uint32_t mlo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)V, 0x140, 0xF, 0xF,
                                                             false);
  const uint32_t mhi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(V >> 32), 0x140,
                                                             0xF, 0xF, false);
  const uint64_t r = xchg64(((uint64_t)mhi << 32) | mlo, 16, ror4_up, lane);
  uint64_t v = L > r ? L : r;
#pragma unroll
  for (int s = 16; s > 0; s >>= 1) {
    const uint64_t o = xchg64(v, s, ror4_up, lane);
    v = (lane & s) == 0 ? (v > o ? v : o) : (v < o ? v : o);
  }
  return v;
}

__device__ __forceinline__ uint64_t ld_coh64(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_coh32(const int32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh64(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh32(int32_t *p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Keys stream through buf (LDS, 128 keys) 64 lanes at a time: lanes with q
// set append their key, and every full 64 are sorted and merged into L.
// The wavefront is alone in its workgroup and its LDS accesses execute in
// order, so only the compiler's ordering is fenced.
struct TopFeed {
  uint64_t *buf;
  uint64_t L = 0;
  int cnt = 0;   // keys waiting in buf (uniform)
  __device__ __forceinline__ void add(uint64_t k, bool q, bool up, int lane) {
    const uint64_t m = __ballot(q);
    if (q) buf[cnt + __popcll(m & ((1ull << lane) - 1))] = k;
    cnt += __popcll(m);
    if (cnt >= 64) {
      asm volatile("" ::: "memory");
      L = merge32v(L, sort64(buf[lane], up, lane), up, lane);
      const uint64_t rest = lane + 64 < cnt ? buf[lane + 64] : 0;
      asm volatile("" ::: "memory");
      buf[lane] = rest;
      cnt -= 64;
    }
  }
  __device__ __forceinline__ uint64_t finish(bool up, int lane) {
    asm volatile("" ::: "memory");
    if (cnt > 0) L = merge32v(L, sort64(lane < cnt ? buf[lane] : 0, up, lane), up, lane);
    asm volatile("" ::: "memory");
    return L;
  }
};

// Top 32 of the wavefront's 1024 keys, 16 per lane (0 = no key), descending
// in lanes 0..31.  The 32nd largest of the 64 lane maxima, tau, bounds the
// 32nd largest key from below (32 distinct keys are >= tau): only keys
// >= tau are merged.
__device__ uint64_t top32_chunk(const uint64_t (&k)[kTkPerLane], uint64_t *buf, bool up,
                                int lane) {
  uint64_t mx = 0;
#pragma unroll
  for (int t = 0; t < kTkPerLane; ++t) mx = k[t] > mx ? k[t] : mx;
  const uint64_t tau = lane_u64(sort64(mx, up, lane), kTk - 1);
  TopFeed f{buf};
#pragma unroll
  for (int t = 0; t < kTkPerLane; ++t) f.add(k[t], k[t] != 0 && k[t] >= tau, up, lane);
  return f.finish(up, lane);
}

// Top 32 of nl <= 16 published lists (32 keys each, descending) at lists:
// pairs of lists load as bitonic sequences (the second reversed), each pair
// is merged, then a tree of merges.  All loads are issued before the first
// is used, and the eight pair merges are independent chains that the
// wavefront interleaves.
__device__ uint64_t top32_lists(const uint64_t *lists, int nl, bool up, int lane) {
  if (nl == 0) return 0;
  uint64_t v[8];
  const int e = lane < kTk ? lane : 63 - lane;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int j = 2 * p + (lane >= kTk ? 1 : 0);
    v[p] = j < nl ? ld_coh64(lists + j * kTk + e) : 0;
  }
#pragma unroll
  for (int p = 0; p < 8; ++p)
    if (2 * p < nl) v[p] = bmerge64(v[p], up, lane);
#pragma unroll
  for (int w = 1; w < 8; w <<= 1)
#pragma unroll
    for (int p = 0; p < 8; p += 2 * w)
      if (2 * (p + w) < nl) v[p] = merge32v(v[p], v[p + w], up, lane);
  return v[0];
}

constexpr uint32_t kTkSpin = 1u << 20;   // polls before a wait gives up

// every word w[0..cnt) satisfies pred (bounded; false if it gave up)
template <typename Pred>
__device__ bool wait_words(const int32_t *w, int cnt, Pred pred, int lane, uint32_t spin) {
  for (uint32_t it = 0; it < spin; ++it) {
    bool ok = true;
    for (int j = lane; j < cnt; j += 64) ok = ok && pred(ld_coh32(w + j));
    if (__all(ok)) return true;
    __builtin_amdgcn_s_sleep(2);
  }
  return false;
}

// Rows of chunk c: [chunk_first(c), chunk_first(c) + chunk_rows(c)) within n.
__device__ __forceinline__ int64_t chunk_first(int c) {
  return c == 0 ? 0 : kTkFirst + (int64_t)(c - 1) * kTkRows;
}
__device__ __forceinline__ int64_t chunk_end(int c, int64_t n) {
  const int64_t e = c == 0 ? kTkFirst : chunk_first(c) + kTkRows;
  return n < e ? n : e;
}

// Chunk c's part of the scan, by one wavefront, from its values: yv[t] is
// row chunk_first(c) + lane + 64 t (anything past the chunk's end).  rows
// (kTkRows int32) and buf (128 keys) are this wavefront's LDS.  Flags
// (epoch > 0): pub[c] = epoch once chunk c's list is in part[c]; spub[s] =
// epoch once super-chunk s's list is in sup[s]; done[c] = 2 epoch + (chunk
// c's replay set the overflow bit).  out = vals[32], rows[32], count,
// overflow (entries past count are zero), written by the last chunk.
// Returns false if a wait gave up after `spin` polls.
__device__ bool chunk_run(const int32_t (&yv)[kTkPerLane], int32_t *rows, uint64_t *buf,
                          int64_t n, int nchunks, int c, int32_t epoch, uint64_t *part,
                          uint64_t *sup, int32_t *flags, int32_t *out, uint32_t spin, bool up,
                          int lane) {
  int32_t *pub = flags, *done = flags + kTopkMaxChunks, *spub = flags + 2 * kTopkMaxChunks;
  const int64_t s0 = chunk_first(c);
  const int64_t end = chunk_end(c, n);
  uint64_t keys[kTkPerLane];
#pragma unroll
  for (int t = 0; t < kTkPerLane; ++t) {
    const int64_t r = s0 + lane + 64 * t;
    rows[lane + 64 * t] = yv[t];
    keys[t] = r < end ? tk_key(yv[t], (uint32_t)r) : 0;
  }
  const uint64_t own = top32_chunk(keys, buf, up, lane);
  if (lane < kTk) st_coh64(part + (int64_t)c * kTk + lane, own);
  wait_vm();
  if (lane == 0) st_coh32(pub + c, epoch);
  // the list of the earlier chunks of this super-chunk ...
  const int s = c / kTopkSuper, c0 = s * kTopkSuper;
  auto is_epoch = [epoch](int32_t v) { return v == epoch; };
  bool ok = wait_words(pub + c0, c - c0, is_epoch, lane, spin);
  const uint64_t W = top32_lists(part + (int64_t)c0 * kTk, c - c0, up, lane);
  if (c - c0 == kTopkSuper - 1) {
    const uint64_t S = merge32v(W, own, up, lane);   // all lanes take part in a merge
    if (lane < kTk) st_coh64(sup + s * kTk + lane, S);
    wait_vm();
    if (lane == 0) st_coh32(spub + s, epoch);
  }
  // ... and of the earlier super-chunks: the list before this chunk
  ok = wait_words(spub, s, is_epoch, lane, spin) && ok;
  const uint64_t pre = merge32v(top32_lists(sup, s, up, lane), W, up, lane);
  // replay this chunk's arrivals
  uint64_t L = pre;
  int32_t cv = tk_val(lane_u64(L, kTk - 1));   // entry 31's value (INT32_MIN while empty)
  int ovf = 0;
  for (int64_t g = s0; g < end && !ovf; g += 64) {
    const int64_t r = g + lane;
    const bool in = r < end;
    const int32_t v = in ? rows[r - s0] : 0;
    // rows 0..31 always enter; later rows only at or above entry[31]
    const bool isc = in && (r < kTk || v >= cv);
    uint64_t cand = __ballot(isc);
    if (__popcll(cand) > kTkSerialMax) {
      // Only a row equal to an earlier row still in the list can set the
      // overflow bit.  If no candidate's value equals a list entry's or
      // another candidate's, the group cannot set it, and the list becomes
      // the top 32 of the list and the group in one merge.
      const uint64_t kv = isc ? tk_key(v, (uint32_t)r) : 0;
      const uint64_t srt = sort64(kv, up, lane);
      const uint64_t prv = shift_up1_u64(srt);
      bool tie = lane > 0 && srt != 0 && (uint32_t)(srt >> 32) == (uint32_t)(prv >> 32);
      // (an empty entry matching a value INT32_MIN only sends the group to
      // the exact path below)
      const uint32_t kh = (uint32_t)(kv >> 32), Lh = (uint32_t)(L >> 32);
#pragma unroll 8
      for (int e = 0; e < kTk; ++e)
        tie = tie || (isc && (uint32_t)__builtin_amdgcn_readlane((int)Lh, e) == kh);
      if (!__any(tie)) {
        L = merge32v(L, srt, up, lane);
        cv = tk_val(lane_u64(L, kTk - 1));
        continue;
      }
    }
    while (cand) {
      const int j = __builtin_ctzll(cand);
      cand &= cand - 1;
      const int64_t rj = g + j;
      const int32_t vj = __builtin_amdgcn_readlane(v, j);
      const bool first = rj < kTk;
      if (!first && vj == cv) {
        ovf = 1;   // rejected while equal to entry[31]
        break;
      }
      // insert at pos (64: rejected, nothing moves); branch-free
      const uint64_t kj = tk_key(vj, (uint32_t)rj);
      const uint32_t gt = (uint32_t)__ballot(L > kj);   // entries above kj (lanes 0..31)
      const int pos = first || vj > cv ? __popc(gt) : 64;
      const int32_t e30 = tk_val(lane_u64(L, kTk - 2));
      const uint64_t upv = shift_up1_u64(L);
      L = lane == pos ? kj : (lane > pos ? upv : L);
      cv = pos < kTk - 1 ? e30 : (pos == kTk - 1 ? vj : cv);
    }
  }
  if (c == nchunks - 1) {
    const uint64_t whole = merge32v(pre, own, up, lane);
    ok = wait_words(done, c, [epoch](int32_t v) { return (v >> 1) == epoch; }, lane, spin) && ok;
    int f = ovf;
    for (int j = lane; j < c; j += 64) f |= ld_coh32(done + j) & 1;
    const bool any = __ballot(f != 0) != 0;
    const int count = n < kTk ? (int)n : kTk;
    if (lane < kTk) {
      const bool live = lane < count;
      out[lane] = live ? tk_val(whole) : 0;
      out[kTk + lane] = live ? (int32_t)tk_row(whole) : 0;
    }
    if (lane == 0) {
      out[2 * kTk] = count;
      out[2 * kTk + 1] = any ? 1 : 0;
    }
  } else if (lane == 0) {
    st_coh32(done + c, 2 * epoch + ovf);
  }
  return ok;
}

}  // namespace
}  // namespace tk
}  // namespace w4a8
