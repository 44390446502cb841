/*
 * nssm.h — C ABI of the MI355X (gfx950) Mamba2 decode-step state update with
 * nested hot/cold tiering ("v4").
 *
 * Everything here is plain C: device pointers, sizes and a hipStream_t passed
 * as void*. No torch types. Every entry point enqueues work on `stream`,
 * never synchronises the host, never allocates device memory, and returns 0
 * or a negative NSSM_E* code (nssm_strerror() names it).
 *
 * Notation: b = requests in a call, H heads, P headdim, N d_state (128),
 * G groups (HG = H/G heads per group), K = k_hot (hot columns: 16, 32, 64 or
 * 96; 0 for the teacher-forced readout only), NC = N-K cold columns, c = flush
 * period in tokens.
 *
 * Reference interfaces these entry points replace (files of the reference
 * repository omin-Kwon/nested_ssm):
 *   nssm_fresh_step      scale/bench_v4_decode.py:250-253 (fresh SSU arm) and
 *                        scale/v4_native_decode.py:58-78 (pb >= N branch)
 *   nssm_v4_step         scale/v4_fused_decode.py:28-95 (_v4_fused_decode),
 *                        scale/v4_native_decode.py:58-167 (_v4_decode state
 *                        part), scale/vllm_v4_patch.py:140-179 (decode_readout)
 *   nssm_v4_step_gated   scale/v4_native_decode.py:118-127 (coldoff) and
 *                        :147-156 (qgate) of _v4_decode
 *   nssm_v4_step_teacher scale/nemo9b_eval.py:41-85 (naive_mixer_forward, modes
 *                        "v4" and, with k_hot = 0, "c1": the teacher-forced
 *                        evaluation readout)
 *   nssm_v4_step_teacher_lagged  the same loop with CFG["lag"] = 1
 *                        (scale/nemo9b_eval.py:44,59,70: readers one snapshot
 *                        behind, the asynchronous-flush model)
 *   nssm_v4_join         scale/vllm_v4_patch.py:123-137 (prefill_snapshot),
 *                        scale/v4_native_decode.py:234-243,
 *                        scale/v4_fused_decode.py:121-159 (prefill capture)
 *   nssm_v4_materialize  no single reference function: the exact current
 *                        state that scale/v4_native_decode.py:65-67 keeps in
 *                        the cache, rebuilt from the tiers
 *   nssm_fp8_readout     scale/bench_v4_decode.py:33-60 (_fp8_matvec /
 *                        fp8_cold_readout)
 *   nssm_check_slots     none (device-side slot id check for callers that cannot sync)
 *   nssm_stream_probe    none (a plain streaming read / copy, for HBM rate comparisons)
 *   nssm_rotate          scale/nemotron_retrofit.py:24-27 (ActRotMask._rot),
 *                        scale/vllm_v4_patch.py:41-45 (rot_flat)
 *   nssm_gated_rmsnorm   scale/v4_native_decode.py:170-171 (self.norm(y, gate):
 *                        transformers' Zamba2RMSNormGated of the mixer)
 *   nssm_conv_update     scale/v4_fused_decode.py:37-44 (causal_conv1d_update
 *                        with SiLU and the x / B / C split; causal-conv1d
 *                        1.6.2.post1, restated by transformers'
 *                        modeling_nemotron_h.causal_conv1d_update)
 */
#ifndef NSSM_H_
#define NSSM_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSSM_ABI_VERSION 16

/* error codes */
#define NSSM_OK 0
#define NSSM_E_NULL (-1)        /* a required pointer is NULL            */
#define NSSM_E_DIMS (-2)        /* sizes out of the supported range      */
#define NSSM_E_ALIGN (-3)       /* a pointer is not aligned as required  */
#define NSSM_E_KIND (-4)        /* unknown cold storage kind             */
#define NSSM_E_LAUNCH (-5)      /* the HIP launch reported an error      */
#define NSSM_E_TUNING (-6)      /* launch override does not fit the dims */
#define NSSM_E_WORKSPACE (-7)   /* workspace NULL or too small           */
#define NSSM_E_SCRATCH (-8)     /* the call needs more than NSSM_SCRATCH_BYTES of scratch */

/* Size of the library's fixed per-device scratch array (nssm_v4_step_noalloc). */
#define NSSM_SCRATCH_BYTES (32u << 20)

/* x ring layouts (nssm_tier.x_layout). Row-major: a token's append is one run per head,
 * the layout of the stale readouts. Unit-blocked: the exact readout's per-token window reads
 * are one run per unit, at the cost of appends that write 16 bytes into each unit's line
 * (9B shape, c = 64: exact readout 9.06 -> 8.90 ms per step; stale c = 4 8.48 -> 8.69). Every
 * entry point serves both. */
#define NSSM_XRING_ROW 0
#define NSSM_XRING_UNIT 1

/* model dtypes of the conv prologue's tensors */
#define NSSM_DT_F32 0
#define NSSM_DT_BF16 1

/* cold tier storage kinds */
#define NSSM_COLD_FP32 0 /* one exact fp32 copy, read every token, rewritten at flush */
#define NSSM_COLD_BF16 1 /* bf16 read copy (RNE of the master) + exact fp32 master */
#define NSSM_COLD_FP8 2  /* e4m3fn read copy, fp32 scale per (slot,head,p) row
                            (amax/448 + 1e-12), + exact fp32 master */
#define NSSM_COLD_NONE 3 /* hot tier only: the cold columns are dropped (never stored,
                            read or flushed); cold, scale, master and the ring may be NULL */
#define NSSM_COLD_BF16_SINGLE 4 /* one bf16 copy, read every token and rewritten at flush
                                   with the RNE of the fp32 flush (the bf16 snapshot master of
                                   scale/v4_fused_decode.py:156-158 and the bf16 arm of
                                   scale/bench_v4_decode.py:160-175); no master */
#define NSSM_COLD_FP8_BF16M 5 /* e4m3fn read copy with the per-row scale of NSSM_COLD_FP8,
                                 quantized from a bf16 master (RNE of the fp32 flush): the
                                 bf16 shadow master of scale/v4_fused_decode.py:149 */

/* Per-layer constants. Mirrors the mixer attributes the reference reads:
 * dt_bias, A = -exp(A_log), D, time_step_min, and the ActRotMask R. */
typedef struct nssm_layer_params {
  int32_t H, P, N, G;
  const float* dt_bias; /* [H] */
  const float* A;       /* [H], already -exp(A_log) */
  const float* D;       /* [H] */
  const float* R;       /* [G][N][N], R[g][m][n]; B'[m] = sum_n R[g][m][n] B[n]; NULL = identity */
  float dt_min;         /* dt = max(dt, dt_min) when dt_min > 0 (v4_native_decode.py:55) */
} nssm_layer_params;

/* One decode token for b requests (all bf16, as the model emits them). */
typedef struct nssm_step_inputs {
  int32_t b;
  const uint16_t* x;        /* [b][H][P] bf16 conv/SiLU output, head view; 8-byte aligned */
  const uint16_t* B;        /* [b][G][N] bf16, before rotation */
  const uint16_t* C;        /* [b][G][N] bf16, before rotation */
  const uint16_t* dt;       /* [b][H] bf16, before dt_bias and softplus */
  const int32_t* slot_ids;  /* [b] state slot of each request, unique; NULL = 0..b-1.
                               The step kernels do not check uniqueness: duplicates race
                               on that slot's tier rows, phase and ring (undefined
                               state); nssm_check_slots flags them on the device. An id
                               outside [0, slots) gives NaN rows of y and leaves every
                               slot untouched. */
} nssm_step_inputs;

/* Tiered state of one layer for `slots` sequence slots (all buffers are
 * owned by the caller). Layouts, row-major unless noted:
 *   hot      fp32 [slots][H][P][K]
 *   cold     [slots][H][P][NC]   fp32 | bf16 | e4m3fn bytes, by cold_kind
 *                                (bf16: unit-blocked, below)
 *   scale    fp32 [slots][H][P]         (FP8 and FP8_BF16M, else NULL)
 *   master   [slots][H][P][NC]          fp32 for BF16 / FP8, bf16 for FP8_BF16M
 *                                       (unit-blocked, below), else NULL
 *   ring_x   bf16 [slots][H][c][P]      x of buffered tokens (x_layout NSSM_XRING_ROW), or
 *            [slots][H][P/8][c][8]      unit-blocked (NSSM_XRING_UNIT: a unit's 8 rows at
 *                                       its c ring positions are one contiguous run)
 *   ring_dt  fp32 [slots][H][c]         softplus'd dt of buffered tokens
 *   ring_b   fp32 [slots][G][c][NC]     rotated B cold columns of buffered tokens
 *   t        int32 [slots][H]           decode steps (phase = t % c)
 *   nv       int32 [slots][H]           buffered tokens since the last snapshot
 *   glog     fp32 [slots][H]            log-decay since the snapshot, one token lagged
 * All heads of a slot carry equal t and nv. hot, cold, master, ring_x and ring_b
 * are 16-byte aligned. k_hot = 0 (every column cold; hot may be NULL, it is never
 * read) needs a cold tier and serves nssm_v4_step_teacher(_lagged), join and
 * materialize; the other step entry points return NSSM_E_DIMS for it.
 * Unit-blocked (the bf16 read copies, the bf16 master): with row = (slot H + h) P + p,
 * element (row, col) sits at (row / 8) 8 NC + (col / 32) 256 + (row % 8) w + col % 32,
 * w = min(32, NC - 32 (col / 32)): the 8 rows of a unit form one block, 32-column segment
 * by segment (a trailing 16-column segment when NC = 112), so a wave moves whole cache
 * lines of it (the sizes are those of [slots][H][P][NC]). */
typedef struct nssm_tier {
  int32_t slots, k_hot, c, cold_kind;
  float* hot;
  void* cold;
  float* scale;
  void* master;
  uint16_t* ring_x;
  float* ring_dt;
  float* ring_b;
  int32_t* t;
  int32_t* nv;
  float* glog;
  int32_t x_layout; /* NSSM_XRING_ROW or NSSM_XRING_UNIT (NSSM_E_KIND otherwise) */
} nssm_tier;

/* Byte size of each tier buffer, in the struct's order (hot, cold, scale,
 * master, ring_x, ring_dt, ring_b, t, nv, glog): sizes_out[10]. */
int nssm_tier_sizes(int32_t slots, int32_t H, int32_t P, int32_t N, int32_t G,
                    int32_t k_hot, int32_t c, int32_t cold_kind, int64_t* sizes_out);

/* Bytes of device workspace a step needs for b requests (c = 0 for the
 * untiered step), or a negative NSSM_E* code. The workspace holds the rotated
 * B and C, per-head decay scalars, flush weights and the exact readout's window
 * dots of one call; it is
 * caller-owned, 16-byte aligned, and must not be shared by steps that run
 * concurrently on different streams. */
int64_t nssm_step_workspace_bytes(int32_t b, int32_t H, int32_t G, int32_t N, int32_t c);

/* Untiered decode step over the full fp32 state [slots][H][P][N]:
 *   B',C' = R_g B, R_g C;  dt = softplus(dt + dt_bias);  a = dt*A
 *   S <- exp(a) S + (dt x) (x) B';   y = S C' + D x          (y fp32 [b][H][P]) */
int nssm_fresh_step(const nssm_layer_params* prm, float* state, int32_t slots,
                    const nssm_step_inputs* in, float* y, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* Tiered decode step (hot fresh, cold stale + decay-corrected, ring append,
 * flush for requests whose phase wraps), two kernels on `stream` (three when c > 16,
 * or c > 32 for NSSM_COLD_BF16_SINGLE):
 *   hot  <- exp(a) hot + (dt x) (x) B'[:K]
 *   y    =  hot C'[:K] + exp(glog) * (cold_read C'[K:]) + D x
 *   this token (x, dt, B'[K:]) goes to ring position t % c; t += 1;
 *   if t % c == 0: cold <- exact cold state at t (decayed replay of the nv
 *   buffered tokens and this one onto the snapshot), nv <- 0, glog <- 0;
 *   else nv += 1, glog += a. */
int nssm_v4_step(const nssm_layer_params* prm, const nssm_tier* tier,
                 const nssm_step_inputs* in, float* y, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* nssm_v4_step for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc). No counterpart in the
 * reference: the same kernels and results as nssm_v4_step, but the per-call workspace is
 * the library's own file-scope device array of NSSM_SCRATCH_BYTES (32 MiB), one per GPU,
 * held until the process ends (its address is looked up once per device, on the first
 * call made with that device current). The call allocates nothing and returns
 * NSSM_E_SCRATCH when nssm_step_workspace_bytes(b, H, G, 128, c) exceeds
 * NSSM_SCRATCH_BYTES (at H = 128, G = 8: up to 2028 requests at c = 4, 1055 at c = 32,
 * 682 at c = 64). Nothing in the scratch needs to start at zero (every word a later
 * kernel reads is written earlier in the same call). Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (different streams, or host threads
 * enqueueing concurrently on one device) race on it; calls ordered on one stream do not. */
int nssm_v4_step_noalloc(const nssm_layer_params* prm, const nssm_tier* tier,
                         const nssm_step_inputs* in, float* y, void* stream);

/* nssm_v4_step with the rank-c exact correction readout instead of the stale
 * one: replaces `_v4_decode` with v4cfg["corr"] = 1 (scale/v4_native_decode.py:81-117).
 * With G = glog + a (inclusive of this token) and the window j = 0..nv (the
 * buffered tokens, then this one),
 *   y = hot C'[:K] + exp(G) (cold_read C'[K:])
 *       + sum_j exp(sum_{i>j} a_i) dt_j (C'[K:] . B'_j[K:]) x_j + D x,
 * which is the current cold state's readout for an fp32 cold tier. The tier
 * bookkeeping (ring, t, nv, glog, flush) is nssm_v4_step's, so calls of the two
 * may alternate on one tier. NSSM_E_KIND for NSSM_COLD_NONE (no cold tier). */
int nssm_v4_step_exact(const nssm_layer_params* prm, const nssm_tier* tier,
                       const nssm_step_inputs* in, float* y, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* nssm_v4_step with the teacher-forced v4 readout of scale/nemo9b_eval.py:41-85 (the
 * per-token evaluation forward, mode "v4", lag 0): the snapshot is the cold state after
 * the update of a flush token, read at that token without decay, and after it with the
 * decay inclusive of the current token,
 *   flush token:  y = hot C'[:K] + (new cold read copy) C'[K:] + D x
 *   other tokens: y = hot C'[:K] + exp(glog + a) (cold_read C'[K:]) + D x.
 * The reference snapshots at sequence positions t % c == 0 counted from 0: join a
 * sequence's start (its state, zeros from scratch) with phase c - 1 so that its flush
 * tokens are those. The tier bookkeeping is nssm_v4_step's, so the readouts may
 * alternate on one tier. With k_hot = 0 every column is read from the snapshot: the
 * loop's mode "c1" (scale/nemo9b_eval.py:79-80),
 *   y = exp(glog + a) (cold_read C') + D x   (the new read copy at a flush token).
 * NSSM_E_KIND for NSSM_COLD_NONE. */
int nssm_v4_step_teacher(const nssm_layer_params* prm, const nssm_tier* tier,
                         const nssm_step_inputs* in, float* y, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* The lagged snapshot of a tier (caller-owned):
 *   cold   the read copy of the snapshot before the tier's last one: cold's dtype and
 *          layout and size, 16-byte aligned
 *   scale  its fp32 row scales [slots][H][P] (FP8 and FP8_BF16M, else NULL)
 *   wlog   fp32 [slots][H]: the log-decay between that snapshot and the tier's last
 * At a join both snapshots are the joined state: a caller copies the tier's cold (and
 * scale) rows of the joined slots into these and zeroes their wlog. */
typedef struct nssm_lag {
  void* cold;
  float* scale;
  float* wlog;
} nssm_lag;

/* nssm_v4_step_teacher with the evaluation loop's lag = 1 (scale/nemo9b_eval.py:44,59,70):
 * the readout is of the snapshot before the last one, decayed from it,
 *   flush token:  y = hot C'[:K] + exp(w) (old read copy C'[K:]) + D x, w = the
 *                 log-decay of the window this token closes; the old read copy then
 *                 becomes the lagged one (lag->cold, lag->scale) and lag->wlog = w
 *   other tokens: y = hot C'[:K] + exp(glog + a + wlog) (lag->cold C'[K:]) + D x.
 * The tier evolves as with nssm_v4_step; only these steps keep `lag` current, so a tier
 * read this way takes this readout on every step. k_hot = 0 is mode "c1" with lag = 1.
 * NSSM_E_KIND for NSSM_COLD_NONE. */
int nssm_v4_step_teacher_lagged(const nssm_layer_params* prm, const nssm_tier* tier,
                                const nssm_lag* lag, const nssm_step_inputs* in, float* y,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* nssm_v4_step with a gated stale readout: a skipped head's y is hot C'[:K] + D x
 * (no cold term) and, when it does not flush at this token, its cold columns are not
 * read. hot_only != 0 skips every head: the draft readout of v4cfg["coldoff"] = 1
 * (scale/v4_native_decode.py:118-127). Otherwise qgate_tau > 0 skips the heads with
 *   rho = sum_{n>=K} C'_n^2 / max(sum_n C'_n^2, 1e-9) < qgate_tau
 * (v4cfg["qgate"], scale/v4_native_decode.py:147-156), and when counts (device, two
 * int64, 8-byte aligned) is not NULL, counts[0] += the gated heads (b H) and counts[1]
 * += the heads that kept the cold term, by device atomics in stream order. hot_only = 0
 * and qgate_tau = 0 is nssm_v4_step. The tier's bookkeeping is nssm_v4_step's in every
 * case (the reference's coldoff branch advances only t). NSSM_E_DIMS for a NaN or
 * infinite qgate_tau (a negative one gates nothing). */
int nssm_v4_step_gated(const nssm_layer_params* prm, const nssm_tier* tier,
                       const nssm_step_inputs* in, float* y, void* workspace,
                       int64_t workspace_bytes, int32_t hot_only, float qgate_tau,
                       int64_t* counts, void* stream);

/* Capture a tier from full fp32 states [b][H][P][N] into slot_ids[b] (NULL =
 * 0..b-1): hot = S[..,:K], cold = S[..,K:] (rounded to the master's precision,
 * then quantized to the read copy),
 * t = phase[i] (NULL = 0), nv = 0, glog = 0. */
int nssm_v4_join(const nssm_layer_params* prm, const nssm_tier* tier, const float* state,
                 int32_t b, const int32_t* slot_ids, const int32_t* phase, void* stream);

/* Rebuild the exact current full fp32 state [b][H][P][N] of slot_ids[b]:
 * hot as stored; cold = exp(sum a) master + decayed replay of the nv buffered
 * tokens. The tier is not modified. */
int nssm_v4_materialize(const nssm_layer_params* prm, const nssm_tier* tier, float* state_out,
                        int32_t b, const int32_t* slot_ids, void* stream);

/* y[r][p] = sum_n q[r][n] * scale[r][n] * e4m3fn(s8[r][n][p]); rows x nc x pd. */
int nssm_fp8_readout(const float* q, const uint8_t* s8, const float* scale, float* y,
                     int32_t rows, int32_t nc, int32_t pd, void* stream);

/* out[t][g][m] = sum_n R[g][m][n] * in[t][g][n]; in bf16, out fp32. */
/* Duplicate and out-of-range slot ids of one call, found on the device with no host sync
 * (no counterpart in the reference, whose callers own one slot per sequence: it is for
 * callers that cannot synchronise to check slot_ids on the host before a step, join or
 * materialize; the kernels themselves do not check uniqueness). Enqueue it on the call's
 * stream with the call's slot_ids [b]; owner: int64 [slots], 8-byte aligned; state: int32
 * [2]; both zero before the first check and then left to this function. state[1] gets bit
 * 0 when two requests of one call name the same slot and bit 1 when an id is outside
 * [0, slots); the bits stay set until the caller clears them (read state[1] after a sync,
 * outside graph capture). Each check (a graph replay too) uses a tag of its own, kept in
 * state[0]. One workgroup; b up to 2^31 - 1. */
int nssm_check_slots(const int32_t* slot_ids, int32_t b, int32_t slots, int64_t* owner, int32_t* state,
                     void* stream);

int nssm_rotate(const uint16_t* in, const float* R, float* out, int32_t T, int32_t G, int32_t N,
                void* stream);

/* One decode token's causal depthwise conv1d update + SiLU (the mixer's
 * prologue before the state op) and the x / B / C split, one launch:
 *   conv_state[r][c] <- [conv_state[r][c][1:], hbc[r][c]]          (width W <= 8)
 *   u[r][c] = silu(bias[c] + sum_w conv_state[r][c][w] weight[c][w]) (* mask[r])
 *   x_out = u[:, :I] [b][I], B_out = u[:, I:I+GN], C_out = u[:, I+GN:] [b][GN], bf16
 * hbc, conv_state [b][dim][W], weight [dim][W] and bias [dim] (NULL: none) are in
 * `dtype` (NSSM_DT_F32 / NSSM_DT_BF16; in bf16 the conv and the SiLU outputs are
 * rounded to bf16, as torch computes them in that dtype); hbc rows are hbc_stride
 * elements apart (a slice of the in_proj output); mask NULL = 1; dim = I + 2 GN.
 * Width 4: conv_state and weight 16-byte (fp32) / 8-byte (bf16) aligned. */
int nssm_conv_update(int32_t b, int32_t dim, int32_t width, int32_t dtype, const void* hbc,
                     int64_t hbc_stride, void* conv_state, const void* weight, const void* bias,
                     const float* mask, int32_t I, int32_t GN, uint16_t* x_out, uint16_t* B_out,
                     uint16_t* C_out, void* stream);

/* The mixer's epilogue before out_proj, one launch: y (fp32 [b][I], D x included)
 * cast to the model dtype, gated by silu(gate), RMS-normalised per group of gs
 * channels and scaled by weight (transformers' Zamba2RMSNormGated):
 *   v = dtype(y) * silu(gate)  (fp32);  out = weight * dtype(v * rsqrt(mean_group(v^2) + eps))
 * gate rows are gate_stride elements apart (a slice of the in_proj output); gate,
 * weight [I] and out [b][I] in `dtype` (NSSM_DT_F32 / NSSM_DT_BF16); gs <= 2048. */
int nssm_gated_rmsnorm(int32_t b, int32_t I, int32_t gs, int32_t dtype, const float* y,
                       const void* gate, int64_t gate_stride, const void* weight, float eps,
                       void* out, void* stream);

/* Measurement aid, no counterpart in the reference: one launch of a plain streaming
 * kernel over `bytes` of device memory on `stream`, the HBM rate the state op is
 * compared with on the same device. mode 0 reads src (dst: 16 writable bytes, written
 * only when the sum of what was read is +inf); mode 1 copies src to dst. src and dst 16-byte
 * aligned (NSSM_E_ALIGN); bytes a positive multiple of 16384 (NSSM_E_DIMS). */
int nssm_stream_probe(const void* src, void* dst, int64_t bytes, int32_t mode, void* stream);

/* Launch-shape override for the stream kernel (0 = automatic): units (waves, each
 * streaming 8 headdim rows of one head) per workgroup, at most 4; a step returns
 * NSSM_E_TUNING when it does not divide P/8. Process-wide; for tuning sweeps. */
int nssm_set_launch(int32_t units_per_wg);

/* Host-side (CPU) conversions used by the kernels, exported so the CPU test
 * suite can compare them bit for bit with torch's casts. */
void nssm_host_f32_to_e4m3fn(const float* in, uint8_t* out, int64_t n);
void nssm_host_e4m3fn_to_f32(const uint8_t* in, float* out, int64_t n);
void nssm_host_f32_to_bf16(const float* in, uint16_t* out, int64_t n);

const char* nssm_strerror(int code);
int nssm_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* NSSM_H_ */
