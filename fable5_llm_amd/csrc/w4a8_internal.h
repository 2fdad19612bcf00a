// Internal declarations shared by the kernels (w4a8_kernels.hip) and the
// C ABI (w4a8_abi.hip).  Not installed; the public surface is
// include/fable5_w4a8.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a8 {

// ---------------------------------------------------------------------------
// Device weight layout ("tile layout").
//
// Rows are grouped into tiles of 16.  A tile is a sequence of scale blocks;
// block b covers groups 8b..8b+7 (a group is 128 weights of one row, the
// unit that shares one uint16 scale mantissa) and is laid out as
//
//   [scales: 16 rows x 16 B = m[r][8b..8b+7] as uint16 LE, zero padded]
//   [group 8b  : 16 rows x 64 B]
//   [group 8b+1: 16 rows x 64 B] ...
//
// Inside a group chunk, bytes [64r + 16q, 64r + 16q + 16) hold weights
// k = 128g + 32q + [0, 32) of row r, so lane (4r + q) of a wavefront reads
// one contiguous 16-byte piece and a whole wavefront reads the 1 KiB chunk
// with one coalesced load.  Each 32-bit word of a piece covers k0..k0+7:
// byte i carries ((w[k0+i] + 8) & 15) in its low nibble (offset form) and
// (w[k0+4+i] & 15) in its high nibble (two's complement), so
//   (word & 0x0F0F0F0F) are 4 unsigned weights + 8 against x8[k0..k0+3]
//   (word & 0xF0F0F0F0) are 4 signed weights * 16  against x8[k0+4..k0+7]
// and sdot4 consumes both without any further unpacking.  The +8 offset is
// removed exactly with a per-(group, quarter) correction 8 * sum x8[lo k].
//
// Bytes per row = K/2 + 16*ceil(NG/8): identical to the row image's
// K/2 + 64*ceil(NG/32) whenever NG % 32 == 0 (K = 4096, 8192, 12288).
// ---------------------------------------------------------------------------
constexpr int kTileRows = 16;
constexpr int kGroup = 128;
constexpr int kGroupsPerBlock = 8;
constexpr int kScaleChunk = kTileRows * 16;                     // 256
constexpr int kGroupChunk = kTileRows * 64;                     // 1024
constexpr int kBlockBytes = kScaleChunk + kGroupsPerBlock * kGroupChunk;  // 8448
constexpr int kKMax = 12288;     // ng <= 96, the engine envelope
constexpr int kNgMax = kKMax / kGroup;
constexpr int kMaxJobs = 6;
constexpr int kWG = 256;         // threads per workgroup (4 wavefronts)
constexpr int kWaves = kWG / 64;

// PRO_EMUL_DYNQ8 (the FFN block's down projection): x16 = clip16(rs(x2 * x,
// 12)) with x int16 (SILU32 of the gate) and x2 int32 (the up projection),
// i.e. ALU EMUL32 at p0 = 12, then DYNQ8.
enum Prologue { PRO_X8 = 0, PRO_DYNQ8 = 1, PRO_RMSNORM_DYNQ8 = 2, PRO_EMUL_DYNQ8 = 3 };
// EPI_MOVY_I16_ADD: EPI_MOVY_I16 into out (when set), and
// clip16(res[row] + that) into res_out (ALU ADD, the block's residual).
// EPI_TOPK (persistent plans' TOPK-32 head): the raw y32 of each row as an
// 8-byte word {y32, the site's stamp} at (uint64_t *)out + row, for the
// TOPK-32 scan that runs in the same launch.
enum Epilogue {
  EPI_Y32 = 0, EPI_MOVY_I16 = 1, EPI_MOVY_P32 = 2, EPI_SILU32 = 3,
  EPI_SHIFT_I64 = 4, EPI_ARGMAX = 5, EPI_MOVY_I16_ADD = 6, EPI_TOPK = 7
};
constexpr int kEmulP0 = 12;   // EMUL32's shift in the SwiGLU block

struct Layout {
  int32_t K, NG, nblk;
  int64_t tile_bytes;
};

inline Layout layout_for(int32_t K) {
  Layout L;
  L.K = K;
  L.NG = K / kGroup;
  L.nblk = (L.NG + kGroupsPerBlock - 1) / kGroupsPerBlock;
  L.tile_bytes = (int64_t)L.nblk * kScaleChunk + (int64_t)L.NG * kGroupChunk;
  return L;
}

// Weight bytes are read exactly once per pass: non-temporal loads keep them
// from displacing activations, outputs and counters in the caches (a plain
// 4 GiB stream: 6.1 TB/s with ordinary loads, 7.0 TB/s non-temporal).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kAuxNt = 2;   // cache-policy operand of the buffer-load builtins: nt
__device__ __forceinline__ uint4 ldg16_nt(const uint8_t *p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// RMSNorm output binary point.  Within 0..40 the reference's int64 steps
// (x * r << (e - 30) for e > 30, layer_fixed.py:1274) never wrap: |x * r| <
// 2^46 and e - 30 <= 17, so the kernels' 64-bit magnitudes are exact.
// Larger in_f (no 16-bit activation format has one) would make the
// reference's numpy shift wrap, so the engine refuses them.
constexpr int kRmsInFMax = 40;

// Table offsets inside the device table buffer (int32 entries).
constexpr int kRsqrtOff = 0;      // 512 Q1.15 seeds
constexpr int kSigmoidOff = 512;  // 257 Q15 knots
constexpr int kTableLen = 512 + 257;

struct GemvJob {
  const uint8_t *w;   // tile layout
  void *out;
  int32_t nrows;
  int32_t tile0;      // first global tile index of this job
  int32_t sh;
  int32_t epi;
  int32_t p0;         // epilogue shift = p0 - e_x
  int32_t pad_;
  const int16_t *res;   // EPI_MOVY_I16_ADD: residual input
  int16_t *res_out;     // EPI_MOVY_I16_ADD: residual output (stream_kernel: an
                        // EPI_MOVY_I16 job with res_out set adds the residual)
  uint64_t *stamped;    // persistent stream, int16 outputs read by a later site
                        // through stamped words: word i = rows 2i, 2i+1 (low 32
                        // bits) and the producing site's stamp (high 32 bits)
};

// A site.  The fields the weight loops read for every block come first,
// in one 64-byte line (with each job's first tile, job_of's table), so that
// a site's table entry costs its loops two scalar-cache lines, not seven.
struct GemvParams {
  int32_t njobs;
  int32_t total_tiles;
  int32_t K, NG, nblk;
  int32_t tile_rot;         // persistent stream: first tile of WG r is (r + tile_rot) % G
  int64_t tile_bytes;
  int32_t tile0[kMaxJobs];  // job[j].tile0
  int32_t pro;
  int32_t tiles_q, tiles_r; // persistent stream: total_tiles = tiles_q * G + tiles_r
  GemvJob job[kMaxJobs];
  const void *x;            // int8[K] or int16[K]
  const int16_t *norm_w;    // int16[K] Q14 (RMSNorm)
  int32_t in_f, one_plus, e_x_given;
  int32_t fence;            // persistent stream: every earlier site completes on all
                            // workgroups before this one reads its activations
  int32_t fence_at;         // persistent stream: the last fenced site <= this one (0: none)
  int32_t local_pro;        // persistent stream: every workgroup computes this site's
                            // prologue itself, after the wait for site fence_at
                            // (exports by workgroup site % G), instead of copying it
                            // from the staging area
  int32_t stamp_src;        // persistent stream: x is read through stamped words
                            // written by site stamp_src (x_stamped), instead of after
                            // a grid-wide wait; -1: not
  const uint64_t *x_stamped;  // ... the words holding x[0..K) (K / 2 of them)
  uint64_t *prod_stamped;   // persistent stream, a site of two int16 / int32 jobs of
                            // equal rows (a gate and an up projection): the stamped
                            // words of EMUL32(job 1, job 0; 12), formed as the
                            // control wavefront stores job 1's tiles (a workgroup
                            // holds the same tiles of both jobs: tiles per job are a
                            // multiple of the grid, at most kPairTiles per workgroup)
  int8_t *x8_out;           // optional (written by workgroup 0)
  int32_t *e_x_out;         // optional
  int16_t *xn_out;          // optional RMSNorm output
  const int32_t *tables;    // kTableLen entries
  int32_t *err;             // bit 0: y32 overflow; bit 2: an LDS wait gave up
  uint64_t *partials;       // EPI_ARGMAX: one key per workgroup
  const int32_t *x2;        // PRO_EMUL_DYNQ8: int32[K]
  // (a whole number of 64-byte lines: in a site table, every entry's first
  // line is its own)
};
static_assert(sizeof(GemvParams) % 64 == 0, "site table entries start on a line");

// launchers (all asynchronous on `s`)
hipError_t launch_fill_i32(int32_t *p, int32_t v, int64_t n, hipStream_t s);
// reads nbytes (a multiple of 16) of buf once; sink: grid words.  start /
// stop (optional) are recorded by the dispatch itself
hipError_t launch_read(const void *buf, int64_t nbytes, uint32_t *sink, int grid,
                       hipStream_t s, hipEvent_t start, hipEvent_t stop);
hipError_t launch_repack(const uint8_t *img, int64_t nrows, const Layout &L,
                         int64_t stride, uint8_t *dst, hipStream_t s);
hipError_t launch_unpack(const uint8_t *src, int64_t nrows, const Layout &L,
                         int64_t stride, uint8_t *img, hipStream_t s);
hipError_t launch_gemv(const GemvParams &p, int grid, hipStream_t s);
// same launch bracketed by events recorded by the dispatch itself
hipError_t launch_gemv_timed(const GemvParams &p, int grid, hipStream_t s,
                             hipEvent_t start, hipEvent_t stop);
// Persistent decode-step kernel: every site of a plan in one launch of one
// workgroup per CU (8 weight wavefronts holding their next two blocks in
// registers, 1 control wavefront, 3 prologue wavefronts); a site with
// `fence` set waits for one completion flag per workgroup.
constexpr int kStreamNormKMax = 4096;   // RMSNorm sites of a persistent plan
constexpr int kPairTiles = 8;           // tiles per job and workgroup of a paired site
struct StreamParams {
  const GemvParams *sites;  // device array, nsites entries
  int32_t nsites;
  int32_t head_site;        // index of the LM-head site, or -1
  uint32_t *done;           // stream_counter_words(grid, nsites) words, zero when
                            // allocated and never cleared between launches:
                            // a completion flag per workgroup (launch `epoch` stores
                            // (epoch - 1) * (nsites + 1) + s + 1 after site s), one flag
                            // per site whose activations are staged (stores epoch), then
                            // the head's key and arrival count (stream_head_word0)
  uint32_t epoch;           // launches since `done` was zeroed, this one included:
                            // every flag value it stores exceeds all earlier ones;
                            // site s of this launch stamps its words
                            // (epoch - 1) * (nsites + 1) + s + 1
  int8_t *stage;            // nsites * kStageBytes: each site's x8, corrections, e_x
  int32_t *err;             // bit 1: a completion wait gave up; bit 2: an LDS wait did
  int32_t *result;          // head: (index, value) of the maximum, written by the
                            // workgroup that arrives last
  uint64_t *trace;          // optional: nsites + 1 wall-clock stamps taken by
                            // workgroup 0 as it starts each site, and at its end
  uint32_t grid_spin;       // polls before a wait for other workgroups gives up
                            // (err bit 1); 0: the kernel's default
  uint32_t lds_spin;        // ... a wait within the workgroup (err bit 2); 0: default
  // A TOPK-32 head (the last site, EPI_TOPK; head_site is then -1): its rows'
  // stamped words (topk_rows of them), the chunk and super-chunk lists
  // (topk_scratch_bytes), the scan's flags (kTopkFlagWords, compared with
  // epoch, which stays below kTopkEpochMax) and the result vals[32],
  // rows[32], count, overflow; topk_out null: no TOPK-32 head
  const uint64_t *topk_y;
  uint64_t *topk_lists;
  int32_t *topk_flags;
  int32_t *topk_out;
  int32_t topk_rows;
};
// one workgroup per CU; `cooperative`: through the cooperative launch API.
// `dependent`: the kernel built for plans with dependent sites (any site
// with local_pro, stamp_src >= 0 or PRO_EMUL_DYNQ8); the other one leaves
// that code out, and is what plans of independent sites run.
// start / stop (optional) bracket the kernel: recorded by the dispatch itself
// for the plain launch, around it for the cooperative one
hipError_t launch_stream(const StreamParams &sp, int grid, hipStream_t s, bool cooperative,
                         bool dependent, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
int stream_max_blocks_per_cu();
// uint32 words of flags a grid of `grid` workgroups running nsites sites needs
size_t stream_counter_words(int grid, int nsites);
// index of the first site flag
__host__ __device__ inline size_t stream_flag_site0(int grid) {
  return (size_t)(grid + 63) / 64 * 64;
}
// index of the head's words: the uint64 key of the maximum so far (two words),
// then the count of workgroups that have added theirs; both zero between launches
__host__ __device__ inline size_t stream_head_word0(int grid, int nsites) {
  return stream_flag_site0(grid) + (size_t)(nsites + 63) / 64 * 64;
}
// one site's staged activations: x8[kKMax], int32 corrections[kKMax / 32], e_x
constexpr int kStageBytes = kKMax + kKMax / 8 + 16;

hipError_t launch_argmax_final(const uint64_t *partials, int n,
                               int32_t *result, hipStream_t s);
hipError_t launch_rshift_round(const int64_t *v, int64_t n, int s,
                               int64_t *out, hipStream_t st);
hipError_t launch_movy(const int32_t *y, int64_t n, int shift, int mode,
                       void *out, hipStream_t s);
hipError_t launch_alu(int op, const int32_t *y, const int16_t *b, int64_t n,
                      int p0, const int32_t *tables, void *out, hipStream_t s);
// TOPK-32 of n head values y, 1 <= n <= 2^18 (w4a8_topk.hip): out =
// vals[32], rows[32], count, overflow.  scratch: topk_scratch_bytes(n)
// bytes, no initial contents.  flags: kTopkFlagWords words, zero or left
// by earlier launches whose epochs were all below epoch (0 < epoch < 2^29).
constexpr int kTopkSuper = 16;        // chunks per super-chunk
constexpr int kTopkMaxChunks = 17 * kTopkSuper;   // 2^18 rows: 256 + 1 chunks
constexpr int kTopkFlagWords = 2 * kTopkMaxChunks + kTopkMaxChunks / kTopkSuper;
constexpr int32_t kTopkEpochMax = 1 << 29;
size_t topk_scratch_bytes(int64_t n);
int topk_chunks(int64_t n);   // chunks of the scan over n rows
hipError_t launch_topk32(const int32_t *y, int64_t n, void *scratch, int32_t *flags,
                         int32_t epoch, int32_t *out, int32_t *err, hipStream_t s,
                         uint32_t spin = 0);   // polls before a wait gives up; 0: default
// MOVX: int8 values in int16 words -> x window, tail to a 4-byte word
// zeroed; bit 4 of err for a value outside int8
hipError_t launch_movx(const int16_t *src, int64_t n, int8_t *dst, int32_t *err,
                       hipStream_t s);
hipError_t launch_vec_prologue(const GemvParams &p, hipStream_t s);
// Several matrices for the same B tokens in one batched launch (jobs run
// one after another on each workgroup, the weight stream running on across
// them); at most kMmJobs.
constexpr int kMmJobs = 16;
struct MmJobSpec {
  const uint8_t *w;   // tile layout
  int32_t nrows;
  Layout L;
  int32_t sh;
  const int8_t *x8;   // [B][K]
  int32_t *y32;       // [B][nrows]
};
hipError_t launch_matmul_multi(const MmJobSpec *jobs, int n, int32_t B, int32_t *err,
                               hipStream_t s);
// A matmul plan: up to kMmPlanJobs matrices for the same B tokens in one
// launch, their records in a device table (matmul_job_bytes() each) that
// matmul_plan_prepare writes on the host, with the launch shape in cfg.
constexpr int kMmPlanJobs = 128;
struct MmPlanCfg {
  int32_t B, CT, G, tmx, ctxt, R, nl, slot_bytes;
  size_t lds;
};
size_t matmul_job_bytes();
// ns[j] (out): job j's K slices; a job with ns[j] > 1 needs its reduction
// buffers (zero) bound to its record before the first launch
hipError_t matmul_plan_prepare(const MmJobSpec *jobs, int n, int32_t B, void *table,
                               MmPlanCfg *cfg, int32_t *ns);
// part: int64 [ns][B][nrows], the slices' sums (overwritten by every launch)
void matmul_plan_bind(void *table, int j, int64_t *part);
// The split jobs' finishing records (matmul_finish_bytes() each, at most n)
// from a bound table; returns their count.  launch_matmul_finish, after each
// launch of the plan, adds the slices and stores y32 (max_n: the largest
// B * nrows among them).
size_t matmul_finish_bytes();
int matmul_finish_prepare(const void *table, int n, int32_t B, void *fin);
hipError_t launch_matmul_finish(const void *d_fin, int nf, int64_t max_n, int32_t *err,
                                hipStream_t s);
hipError_t launch_matmul_plan(const void *d_table, int n, const MmPlanCfg &cfg,
                              int32_t *err, hipStream_t s);
hipError_t launch_matmul(const uint8_t *w, int32_t nrows, const Layout &L,
                         int32_t sh, const int8_t *x8, int32_t B,
                         int32_t *y32, int32_t *err, hipStream_t s);
int gemv_max_blocks_per_cu();

}  // namespace w4a8
