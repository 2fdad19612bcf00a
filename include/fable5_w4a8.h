/* fable5_w4a8.h -- C ABI of the MI355X W4A8 matvec engine.
 *
 * Replaces the FPGA matvec datapath of coreyhahn/fable5_llm
 * (rtl/matvec_engine.sv, rtl/matvec_chan.sv, rtl/ddr_rd_streamer.sv and the
 * DYNQ8 / MOVX / MOVY movers of rtl/seq_movers.sv + rtl/vec_alu.sv) and the
 * Python law functions of ref/w4a8_ref.py and ref/fixedpoint.py that define
 * it.  Every result is bit-exact with that integer law.
 *
 * Conventions
 *   - every entry point returns int: W4A8_OK (0) or a negative W4A8_E_*;
 *     w4a8_last_error() gives the message of the calling thread's last error
 *   - host-buffer entry points are synchronous; *_async entry points take
 *     DEVICE pointers and enqueue on the context's stream (see
 *     w4a8_ctx_set_stream); a device-side y32 overflow raised by async work
 *     is reported by the next w4a8_ctx_sync()
 *   - one context per host thread; contexts are not internally locked
 *   - weights are uploaded once as the reference's row image
 *     (ref/w4a8_ref.py:349-370 pack_ddr_rows) and repacked on the device;
 *     group size g = 128 (the 9B engine's only format, matvec_engine.sv:17-34)
 */
#ifndef FABLE5_W4A8_H
#define FABLE5_W4A8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (mirror the reference's assertion classes) ---------- */
#define W4A8_OK           0
#define W4A8_E_SHAPE    (-1) /* K % 128, image size, m shape: w4a8_ref.py:104-105, 147-150, 439-440 */
#define W4A8_E_ENVELOPE (-2) /* ng outside 1..96 or sh outside 0..63: hwmap.py:146-169, matvec_engine.sv:716-719 */
#define W4A8_E_ACC_OVF  (-3) /* |acc| >= 2^31: w4a8_ref.py:285 (unreachable for int4 x int8 codes) */
#define W4A8_E_Y32_OVF  (-4) /* |y32| >= 2^31: w4a8_ref.py:288 "y32 overflow — sh miscomputed" */
#define W4A8_E_HIP      (-5) /* HIP runtime failure */
#define W4A8_E_ARG      (-6) /* null / misaligned pointer, bad handle, bad enum */
#define W4A8_E_RANGE    (-7) /* value outside the law's domain: rmsnorm n not a power of 2 or in_f outside 0..40
                                (layer_fixed.py:1270-1272), vocab > 2^18 (gen_model_script.py:564-565),
                                ALU count > 16383 (gen_layer_script.py:1377-1386) */

/* ---- prologue: how the int8 activation vector is produced ------------- */
#define W4A8_PRO_X8             0 /* x is int8[K] already quantised, e_x supplied by caller */
#define W4A8_PRO_DYNQ8          1 /* x is int16[K]: DYNQ8, fixedpoint.py:24-33 */
#define W4A8_PRO_RMSNORM_DYNQ8  2 /* x is int16[K]: RMSNorm (layer_fixed.py:1242-1278) then DYNQ8 */

/* ---- epilogue: what is written per output row ------------------------- */
#define W4A8_EPI_Y32        0 /* int32 y32 (w4a8_ref.py:254-289) */
#define W4A8_EPI_MOVY_I16   1 /* int16 clip16(rs_s(y32, shift)): MOVY int16 / SHIFT32 (seq_model.py:1027-1050) */
#define W4A8_EPI_MOVY_P32   2 /* int32 clip32(rs_s(y32, shift)): MOVY pairs32 / SHIFT32W */
#define W4A8_EPI_SILU32     3 /* int16 SILU32 (gen_layer_script.py:1409-1413) */
#define W4A8_EPI_SHIFT_I64  4 /* int64 rs_s(y32, shift), no clip: layer_fixed.matvec_to (1224-1236) */
/* shift = p0 - e_x (the MOVY IND_SUB XRF[0] encoding, seq_format.py:771-782).
   MOVY-style shifts are capped as the RTL caps them: right by <= 63, left by
   <= 40 (seq_movers.sv:770-777). */

/* ---- ALU ops (rtl/vec_alu.sv op numbers) ------------------------------- */
#define W4A8_ALU_SHIFT32   1
#define W4A8_ALU_SILU32    6
#define W4A8_ALU_EMUL32    8
#define W4A8_ALU_SHIFT32W  9

/* MOVY modes (seq_model.py MOVY_INT16 / pairs) */
#define W4A8_MOVY_PAIRS32  0
#define W4A8_MOVY_INT16    1

typedef struct w4a8_ctx w4a8_ctx;
typedef struct w4a8_weights w4a8_weights;
typedef struct w4a8_plan w4a8_plan;

const char *w4a8_version(void);
const char *w4a8_last_error(void);

/* ---- context (replaces the board lock + channel CSR block,
 *      sw/board_lock.py, matvec_chan.sv:12-49) -------------------------- */
int w4a8_ctx_create(int32_t device, w4a8_ctx **out);
int w4a8_ctx_destroy(w4a8_ctx *ctx);
/* run on a caller-owned hipStream_t (e.g. torch's current stream); NULL
   restores the context's own stream */
int w4a8_ctx_set_stream(w4a8_ctx *ctx, void *hip_stream);
/* wait for the stream; returns W4A8_E_Y32_OVF if async work overflowed */
int w4a8_ctx_sync(w4a8_ctx *ctx);
/* number of compute units and the default persistent grid of the device */
int w4a8_ctx_info(const w4a8_ctx *ctx, int32_t *num_cu, int32_t *grid);
/* override the GEMV grid size (0 = default); for tuning sweeps */
int w4a8_ctx_set_grid(w4a8_ctx *ctx, int32_t grid);
/* no counterpart in the reference: how many polls the context's later
   persistent-plan and TOPK-32 launches make before a bounded wait gives up
   -- grid_polls for waits on other workgroups (reported at the next sync as
   W4A8_E_HIP, "...wait for other workgroups timed out..."; TOPK-32's
   look-back: "...TOPK-32's wait..."), lds_polls for waits between the
   wavefronts of one workgroup ("a wait between wavefronts ...").  A wait
   that gives up lets its kernel run to its end (results undefined), so a
   caller can exercise these error paths without a hang.  0: the defaults
   (2^18 and 2^20 polls). */
int w4a8_ctx_set_spin_limit(w4a8_ctx *ctx, uint32_t grid_polls, uint32_t lds_polls);
/* the rsqrt seed LUT (512 Q1.15) and sigmoid knots (257 Q15) the device
   uses: fixedpoint.py:42-53 and 128-142 (ROMs roms/rsqrt_rom.hex,
   roms/sigmoid_rom.hex) */
int w4a8_tables(w4a8_ctx *ctx, int32_t *rsqrt512, int32_t *sigmoid257);
/* no counterpart in the reference: the measured HBM read ceiling the
   kernels' roofline fractions can be read against -- n launches, each
   reading the nbytes (a multiple of 16, >= 16) at d_buf once with the
   weight stream's 16-byte non-temporal loads over `grid` workgroups of 256
   threads (0: 8 per CU); ms[i] = kernel time of launch i (dispatch-recorded
   events).  Synchronous. */
int w4a8_read_ceiling(w4a8_ctx *ctx, const void *d_buf, int64_t nbytes, int32_t grid,
                      int32_t n, float *ms);

/* ---- weights (replaces the DDR weight image + WBASE/WBEATS/SHAPE CSRs,
 *      w4a8_ref.py:349-370, matvec_chan.sv:12-49) ----------------------- */
/* img: host row image of nrows rows, stride (K/128 + ceil(K/4096))*64 */
int w4a8_weights_upload(w4a8_ctx *ctx, const uint8_t *img, int64_t nrows,
                        int32_t K, int32_t sh, w4a8_weights **out);
/* same, image already in device memory */
int w4a8_weights_upload_async(w4a8_ctx *ctx, const uint8_t *d_img,
                              int64_t nrows, int32_t K, int32_t sh,
                              w4a8_weights **out);
/* inverse repack to the row image (host buffer of nrows*stride bytes):
   w4a8_ref.py:429-446 unpack_ddr_rows view */
int w4a8_weights_download(w4a8_ctx *ctx, const w4a8_weights *w, uint8_t *img);
int w4a8_weights_info(const w4a8_weights *w, int64_t *nrows, int32_t *K,
                      int32_t *sh, int64_t *device_bytes);
int w4a8_weights_free(w4a8_weights *w);

/* ---- elementwise law (host buffers, synchronous) ---------------------- */
/* w4a8_ref.py:90-99 rshift_round */
int w4a8_rshift_round(w4a8_ctx *ctx, const int64_t *v, int64_t n, int32_t s,
                      int64_t *out);
/* fixedpoint.py:24-33 dyn_quant_i8 */
int w4a8_dynq8(w4a8_ctx *ctx, const int16_t *x16, int32_t n, int8_t *x8,
               int32_t *e);
/* layer_fixed.py:1242-1278 rmsnorm_fx */
int w4a8_rmsnorm(w4a8_ctx *ctx, const int16_t *x16, const int16_t *w_q14,
                 int32_t n, int32_t in_f, int32_t one_plus, int16_t *out);
/* seq_model.py:1027-1050 MOVY: out is int16[n] (INT16) or int32[n] (PAIRS32) */
int w4a8_movy(w4a8_ctx *ctx, const int32_t *y32, int64_t n, int32_t shift,
              int32_t mode, void *out);
/* The same MOVY on device buffers, enqueued on the context stream (the
   .seq MOVY record, seq_model.py:1027-1050; shift already resolved through
   the XRF, seq_format.py:771-782).  d_y32 4-byte aligned; d_out 2-byte
   (INT16) or 4-byte (PAIRS32) aligned. */
int w4a8_movy_async(w4a8_ctx *ctx, const int32_t *d_y32, int64_t n,
                    int32_t shift, int32_t mode, void *d_out);
/* The .seq MOVX record's data move (seq_model.py:929-952): n int8 values
   held in int16 scratch words -> the x window d_x8, the tail up to a 4-byte
   word zeroed (SEQ_ISA B6).  A value outside int8 makes the next sync
   return W4A8_E_RANGE ("MOVX source is not int8-packed"). */
int w4a8_movx_async(w4a8_ctx *ctx, const int16_t *d_src, int64_t n,
                    int8_t *d_x8);
/* gen_layer_script.py:1397-1423 ALU ops on int32 pairs: SHIFT32, SILU32,
   EMUL32 (b = int16[n]) -> int16 out; SHIFT32W -> int32 out */
int w4a8_alu(w4a8_ctx *ctx, int32_t op, const int32_t *y32, const int16_t *b,
             int64_t n, int32_t p0, void *out);

/* ---- matvec (host buffers, synchronous) ------------------------------- */
/* w4a8_ref.py:254-289 matvec_y32 */
int w4a8_matvec_y32(w4a8_ctx *ctx, const w4a8_weights *w, const int8_t *x8,
                    int32_t *y32);
/* prologue -> matvec -> epilogue in one launch.  x: int8[K] (PRO_X8, e_x
   taken from *e_x_io) or int16[K]; norm_w: int16[K] Q14 for
   PRO_RMSNORM_DYNQ8 (one_plus selects vecnorm mode 0 = (1+w) / 1 = w);
   out: per epilogue; x8_out (int8[K]), e_x_io, xn_out (int16[K], RMSNorm
   output) are optional */
int w4a8_matvec_fused(w4a8_ctx *ctx, const w4a8_weights *w, int32_t prologue,
                      const void *x, const int16_t *norm_w, int32_t in_f,
                      int32_t one_plus, int32_t epilogue, int32_t p0, void *out,
                      int8_t *x8_out, int32_t *e_x_io, int16_t *xn_out);
/* LM head: matvec + running argmax (AMAX32, strictly greater => lowest
   index wins ties; gen_layer_script.py:1424-1433, gen_model_script.py:627-643) */
int w4a8_head_argmax(w4a8_ctx *ctx, const w4a8_weights *w, int32_t prologue,
                     const void *x, const int16_t *norm_w, int32_t in_f,
                     int32_t one_plus, int32_t *idx, int32_t *val);
/* batched: y32[b][n] = matvec_y32(w, x8[b][:]) for b < B (int8 MFMA) */
int w4a8_matmul_y32(w4a8_ctx *ctx, const w4a8_weights *w, const int8_t *x8,
                    int32_t B, int32_t *y32);

/* ---- device-pointer variants (async on the context stream) ------------ */
int w4a8_matvec_fused_async(w4a8_ctx *ctx, const w4a8_weights *w,
                            int32_t prologue, const void *d_x,
                            const int16_t *d_norm_w, int32_t in_f,
                            int32_t one_plus, int32_t e_x, int32_t epilogue,
                            int32_t p0, void *d_out, int8_t *d_x8_out,
                            int32_t *d_e_x_out, int16_t *d_xn_out);
/* several matrices sharing one input vector in one launch: the MOVX
   broadcast + MVGO x4 analogue (seq_movers.sv:939-1029) */
int w4a8_site_async(w4a8_ctx *ctx, int32_t nmat,
                    const w4a8_weights *const *w, const int32_t *epilogue,
                    const int32_t *p0, void *const *d_out, int32_t prologue,
                    const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                    int32_t one_plus, int32_t e_x, int8_t *d_x8_out,
                    int32_t *d_e_x_out, int16_t *d_xn_out);
/* d_result: int32[2] = {idx, val} */
int w4a8_head_argmax_async(w4a8_ctx *ctx, const w4a8_weights *w,
                           int32_t prologue, const void *d_x,
                           const int16_t *d_norm_w, int32_t in_f,
                           int32_t one_plus, int32_t e_x, int32_t *d_result);
int w4a8_matmul_y32_async(w4a8_ctx *ctx, const w4a8_weights *w,
                          const int8_t *d_x8, int32_t B, int32_t *d_y32);
/* n <= 16 matrices for the same B tokens in one launch (e.g. a layer's
   gate and up, which share x8): matrix i reads d_x8[i] [B][K_i] and writes
   d_y32[i] [B][nrows_i], each row bit-identical to w4a8_matmul_y32_async of
   that matrix alone.  The weight stream runs on across the matrices instead
   of draining at each launch's end.  No counterpart in the reference's C
   interface (its engine runs one matrix per MVGO). */
int w4a8_matmul_y32_multi_async(w4a8_ctx *ctx, int32_t n,
                                const w4a8_weights *const *w,
                                const int8_t *const *d_x8, int32_t B,
                                int32_t *const *d_y32);
/* A matmul plan: up to 128 matrices for the same B tokens (1..64) in ONE
 * launch per run (e.g. a pass over a model's 96 FFN matrices), each matrix
 * i reading its d_x8 [B][K_i] and writing its d_y32 [B][nrows_i], each row
 * bit-identical to w4a8_matmul_y32_async of that matrix alone.  The first
 * run after an add writes the plan's device table (so run it once before
 * capturing it into a graph); a graph captured before a later add keeps
 * replaying the plan as it was (the buffers it names are freed only by
 * destroy); runs enqueue on the context stream.  The
 * weight stream runs on across every matrix of the plan instead of
 * draining at each launch's end.  No counterpart in the reference (its
 * engine runs one matrix per MVGO, one token at a time). */
typedef struct w4a8_mplan w4a8_mplan;
int w4a8_mplan_create(w4a8_ctx *ctx, int32_t B, w4a8_mplan **out);
int w4a8_mplan_add(w4a8_mplan *plan, const w4a8_weights *w, const int8_t *d_x8,
                   int32_t *d_y32);
int w4a8_mplan_run(w4a8_mplan *plan);
int w4a8_mplan_destroy(w4a8_mplan *plan);

/* ---- TOPK-32 over the LM head -----------------------------------------
 * The layer_topk32 block's contract (docs/SEQ_ISA.md B8): the head's raw
 * y32 (shift 0) scanned in row order after one fresh; the 32 largest
 * values sorted descending, ties in row order (entry 0 == the AMAX32
 * winner); count = min(32, rows); overflow = sticky, set when a row was
 * rejected (list full, not greater than entry 31) while exactly equal to
 * entry 31 (TK_STATUS bit 7).  Entries past count are zero.  Replaces the
 * host's TK_VAL / TK_IDX readback loop; no counterpart in the reference's
 * C interface. */
int w4a8_head_topk32(w4a8_ctx *ctx, const w4a8_weights *w, int32_t prologue,
                     const void *x, const int16_t *norm_w, int32_t in_f,
                     int32_t one_plus, int32_t *vals, int32_t *rows,
                     int32_t *count, int32_t *overflow);
/* the same scan over n <= 2^18 int32 values (an AMAX32 command sequence
   over any region feeds the block, SEQ_ISA.md B8) */
int w4a8_topk32(w4a8_ctx *ctx, const int32_t *y32, int64_t n, int32_t *vals,
                int32_t *rows, int32_t *count, int32_t *overflow);
/* d_out: int32[66] = vals[32], rows[32], count, overflow */
int w4a8_head_topk32_async(w4a8_ctx *ctx, const w4a8_weights *w,
                           int32_t prologue, const void *d_x,
                           const int16_t *d_norm_w, int32_t in_f,
                           int32_t one_plus, int32_t e_x, int32_t *d_out);
/* w4a8_head_topk32_async that allocates nothing: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The head's y32 and TOPK-32's lists live in a static device array of
 * 1.07 MiB per GPU (held until the process ends) instead of the context's
 * chain buffer; heads over 2^18 rows are refused with W4A8_E_RANGE.  Every
 * call on one GPU shares that array, from every context: calls that overlap
 * on one GPU race. */
int w4a8_head_topk32_noalloc_async(w4a8_ctx *ctx, const w4a8_weights *w,
                                   int32_t prologue, const void *d_x,
                                   const int16_t *d_norm_w, int32_t in_f,
                                   int32_t one_plus, int32_t e_x, int32_t *d_out);

/* ---- the SwiGLU FFN block on device buffers ---------------------------
 * One decoder layer's MLP (gen_layer_script.py:2166-2190 mlp_block;
 * layer_fixed.py:1597-1604 mlp_fx), enqueued on the context stream:
 *   x8   = DYNQ8(RMSNorm(x16; norm_w, in_f, one_plus))  (d_norm_w null: DYNQ8(x16))
 *   sg   = SILU32(gate . x8; p0_gate)              int16 Q12, FFN wide
 *   u    = SHIFT32W(up . x8; p0_up)                int32, FFN wide
 *   prod = EMUL32(u, sg; 12)                       int16
 *   y    = SHIFT32(down . DYNQ8(prod); p0_down)    int16, H wide -> d_mlp_out
 *   d_res_out = clip16(x16 + y)                    ALU ADD, the residual add
 * One output may be null (not both); d_res_out may be x16 itself.  p0_*
 * are MOVY immediates (shift = p0 - e_x, as in plan sites).  gate, up:
 * FFN x H; down: H x FFN.  Temporaries (sg, u) live in the context (grown
 * on first use).  2 launches: gate and up share one; the down projection
 * forms EMUL32 in its prologue and the ADD in its epilogue, so prod never
 * reaches memory.  No counterpart in the
 * reference's C interface: it chains the reference's per-record operations
 * (MVGO, the SILU32 / SHIFT32W / EMUL32 / DYNQ8 / ADD ALU ops) on the
 * device. */
int w4a8_mlp_async(w4a8_ctx *ctx, const w4a8_weights *gate,
                   const w4a8_weights *up, const w4a8_weights *down,
                   int32_t p0_gate, int32_t p0_up, int32_t p0_down,
                   const int16_t *d_x16, const int16_t *d_norm_w, int32_t in_f,
                   int32_t one_plus, int16_t *d_mlp_out, int16_t *d_res_out);

/* ---- plans: a fixed sequence of sites (and the LM head) replayed as one
 *      unit -- the record stream of one decode step (MOVX/MVGO/FENCE/MOVY
 *      per site, seq_format.py:2077-2231).  Every result is that of running
 *      the sites one after another.  All pointers are device pointers
 *      captured at add time.  A graph the caller captured from a run stays
 *      valid after later adds (it replays the plan as it was then): the
 *      device buffers of earlier builds are freed only by destroy. ----- */
#define W4A8_PLAN_GRAPH       0 /* one launch per site, replayed as a HIP graph;
                                   site s+1 starts after site s has completed */
#define W4A8_PLAN_PERSISTENT  1 /* one launch for every site, one workgroup
                                   per CU; a fenced site waits for
                                   per-workgroup completion flags, and each
                                   wavefront keeps its next weight blocks in
                                   flight across the wait.  The grid is the
                                   device's CU count and the kernel's LDS
                                   admits one workgroup per CU, so on a GPU
                                   not running other long kernels every
                                   workgroup is resident at once; the waits
                                   between workgroups are bounded, and report
                                   an error (W4A8_E_HIP at the next sync)
                                   instead of hanging where one is not */
#define W4A8_PLAN_PERSISTENT_COOP 2 /* the same launch through the cooperative
                                   launch API, which guarantees that every
                                   workgroup is resident (for a GPU shared
                                   with other long-running kernels); the
                                   runtime's cooperative dispatch costs about
                                   23 us per launch on MI355X */
/* fences of a persistent plan */
#define W4A8_FENCE_ALL   0 /* (default) every site waits for all earlier ones */
#define W4A8_FENCE_AUTO  1 /* a site waits only when it reads a buffer an
                              earlier site (since the last fence) writes, or
                              writes one such a site reads or writes -- byte
                              ranges of x, RMSNorm weights, outputs, x8 / e_x /
                              RMSNorm exports and the head result */
int w4a8_plan_create(w4a8_ctx *ctx, w4a8_plan **out);
int w4a8_plan_add_site(w4a8_plan *plan, int32_t nmat,
                       const w4a8_weights *const *w, const int32_t *epilogue,
                       const int32_t *p0, void *const *d_out, int32_t prologue,
                       const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                       int32_t one_plus, int32_t e_x, int8_t *d_x8_out,
                       int32_t *d_e_x_out, int16_t *d_xn_out);
/* The SwiGLU product site of a decode step (gen_layer_script.py:2166-2190,
   layer_fixed.py:1597-1604): the ALU's EMUL32 of the gate's SILU32 output
   d_x (int16[K]) with the up projection's output d_x2 (int32[K]) at p0 = 12,
   then DYNQ8, then the site's matrices (the down projection) with their
   epilogues.  K is the matrices' K (<= 12288).  The reference runs these as
   the ALU commands between the gate/up MOVYs and the down MVGOs; here they
   are the site's prologue, so the product never reaches memory.  x8 / e_x
   exports as for w4a8_plan_add_site. */
int w4a8_plan_add_site_emul(w4a8_plan *plan, int32_t nmat,
                            const w4a8_weights *const *w, const int32_t *epilogue,
                            const int32_t *p0, void *const *d_out, const int16_t *d_x,
                            const int32_t *d_x2, int8_t *d_x8_out, int32_t *d_e_x_out);
/* The SwiGLU product site with the block's residual ADD: down (H x FFN)
 * over DYNQ8(EMUL32(x2, x; 12)) as w4a8_plan_add_site_emul, MOVY int16 at
 * p0 into d_out (may be null) and clip16(res + that) into d_res_out; the
 * down launch of w4a8_mlp_async (gen_layer_script.py:2166-2190,
 * 1399-1400) as a plan site.  No counterpart in the reference's C
 * interface (its sequencer issues the block as records). */
int w4a8_plan_add_site_emul_res(w4a8_plan *plan, const w4a8_weights *down,
                                int32_t p0, int16_t *d_out, const int16_t *d_x,
                                const int32_t *d_x2, const int16_t *d_res,
                                int16_t *d_res_out);
/* A layer's whole FFN block as two plan sites: w4a8_mlp_async's arguments
 * (layer_fixed.py:1597-1604 mlp_fx), its temporaries owned by the plan.
 * In a persistent plan the gate and up site forms the EMUL32 product as it
 * stores and the down site waits for the product's words. */
int w4a8_plan_add_mlp(w4a8_plan *plan, const w4a8_weights *gate,
                      const w4a8_weights *up, const w4a8_weights *down,
                      int32_t p0_gate, int32_t p0_up, int32_t p0_down,
                      const int16_t *d_x16, const int16_t *d_norm_w, int32_t in_f,
                      int32_t one_plus, int16_t *d_mlp_out, int16_t *d_res_out);
int w4a8_plan_add_head(w4a8_plan *plan, const w4a8_weights *w,
                       int32_t prologue, const void *d_x,
                       const int16_t *d_norm_w, int32_t in_f, int32_t one_plus,
                       int32_t e_x, int32_t *d_result);
/* The LM head ending in TOPK-32 instead of the argmax: the layer_topk32
 * block fed from the AMAX32 compare site in the same pass over the rows
 * (docs/SEQ_ISA.md:582-610; the sampling loop reads it,
 * sw/chat_seq.py:284-291).  d_out: vals[32], rows[32], count, overflow as
 * w4a8_head_topk32_async.  One per plan; in a persistent plan it is the last
 * step and its scan runs inside the same launch, chunk by chunk as the
 * head's rows are stored; in graph mode the head's y32 is followed by the
 * TOPK-32 kernel. */
int w4a8_plan_add_head_topk32(w4a8_plan *plan, const w4a8_weights *w,
                              int32_t prologue, const void *d_x,
                              const int16_t *d_norm_w, int32_t in_f, int32_t one_plus,
                              int32_t e_x, int32_t *d_out);
int w4a8_plan_set_mode(w4a8_plan *plan, int32_t mode);
/* no counterpart in the reference (its sequencer orders every record): how
   a persistent plan orders its sites, W4A8_FENCE_ALL or W4A8_FENCE_AUTO */
int w4a8_plan_set_fences(w4a8_plan *plan, int32_t fences);
/* no counterpart in the reference: how a persistent replay orders site i
   (under the plan's fence mode): fenced[i] = 1 where it waits for every
   workgroup to finish every earlier site, 2 where it waits only for the
   output of one earlier site that it reads as its input (through that
   output's stamped words), 0 where it waits for nothing.  n = number of
   steps.  Host-only, enqueues nothing. */
int w4a8_plan_fences(w4a8_plan *plan, int32_t n, int32_t *fenced);
/* enqueue one replay of the whole plan on the context stream */
int w4a8_plan_run(w4a8_plan *plan);
/* run every step once, each GEMV launch bracketed by dispatch-recorded
   events; ms[i] = kernel time of step i (n = number of steps).  In
   persistent mode the single launch's event-measured time is split over the
   steps by wall-clock stamps taken as workgroup 0 starts each site.
   Synchronous. */
int w4a8_plan_profile(w4a8_plan *plan, int32_t n, float *ms);
/* no counterpart in the reference: n replays of a persistent plan enqueued
   back to back, each launch bracketed by events its dispatch records;
   ms[i] = kernel time of replay i.  Synchronous.  W4A8_E_ARG in graph
   mode (a replay is many launches there: use w4a8_plan_profile). */
int w4a8_plan_time_launches(w4a8_plan *plan, int32_t n, float *ms);
int w4a8_plan_destroy(w4a8_plan *plan);

#ifdef __cplusplus
}
#endif
#endif /* FABLE5_W4A8_H */
