// gfx950 kernels for the Mamba2 decode-step recurrent-state update with
// nested hot/cold tiering, and the C ABI declared in include/nssm.h.
//
// A tiered layer-token is two launches on the caller's stream (prep, stream) when the
// flush window is at most 16 tokens (32 for a single bf16 copy), three beyond (prep,
// stream, flush); the untiered step is prep and stream:
//
//  prep    one workgroup per (group, block of requests). Rotates B and C once
//          (B' = R_g B, C' = R_g C, fp32) into the workspace, computes each
//          head's dt, decay, the stale-read factor exp(glog), the flush flag
//          and, at a flush, the decay weights of the buffered window; updates
//          t, nv, glog; appends this token (dt, B' cold columns) to the ring
//          at position t % c. A flush token sits at c-1, so a flush window is
//          always ring positions [c-m, c).
//  stream  one wave per "unit", 8 consecutive headdim rows p of one head (lane l
//          works on row p0 + (l >> 3), and a row's C.h readout is a sum over its
//          8 lanes, three DPP steps), a few units of one head per workgroup. Hot
//          columns [0, K) are read and written every token; cold columns [K, N)
//          are only read (the stale readout) except by a head that flushes at
//          this token, whose short window is replayed here.
//  flush   (longer windows) the cold columns of the heads that flush:
//          decayed snapshot plus the window contraction on the matrix cores,
//          and their stale readout.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <set>
#include <type_traits>
#include <utility>

#include "../../include/nssm.h"
#include "nssm_formats.h"

namespace {

constexpr int kN = 128;  // d_state handled by these kernels
constexpr int kMaxC = 64;
constexpr int kFusedMaxWindow = 32;  // longest window the stream kernel replays itself
constexpr int kMaxHG = 64;  // heads per group
constexpr int kMaxUnitsPerWg = 4;  // waves (units) per stream workgroup
constexpr int kMfmaTiles = 5;  // 16 x 16 flush-contraction tiles a wave keeps in registers

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

// address-space casts for gfx950's LDS DMA (global_load_lds)
#define NSSM_GLOBAL(p) ((const __attribute__((address_space(1))) void*)(p))
#define NSSM_LOCAL(p) ((__attribute__((address_space(3))) void*)(p))

struct StepArgs {
  // tier state (fresh: hot is the full state, the rest NULL)
  float* hot;
  void* cold;
  float* scale;
  void* master;  // fp32 (bf16 / e4m3 read copies) or bf16 (NSSM_COLD_FP8_BF16M)
  uint16_t* ring_x;
  float* ring_dt;
  float* ring_b;
  int32_t* t;
  int32_t* nv;
  float* glog;
  // inputs
  const uint16_t* x;
  const uint16_t* Bm;
  const uint16_t* Cm;
  const uint16_t* dt_raw;
  const int32_t* slot_ids;
  const float* dt_bias;
  const float* A;
  const float* D;
  const float* R;
  float* y;
  float* ws;  // workspace (see Ws below)
  int32_t b, slots, H, P, G, HG, c, K;
  // x ring layout (NSSM_XRING_*): element (slot H + head, position pos, headdim row p) sits at
  // (slot H + head) c P + pos xs_tok + (p / 8) xs_unit + p % 8, so the 8 rows of a unit at
  // one position are one 16-byte granule in either layout
  int32_t xs_tok, xs_unit;
  int32_t prb;    // requests per prep workgroup
  int32_t exact;  // rank-c exact correction readout instead of the stale one
  int32_t tf;     // teacher-forced readout: inclusive decay; a flushing head reads its new state
  int32_t split;  // the flush kernel runs after the stream kernel (prep writes the pair flags)
  int32_t fch;    // window tokens the flush kernel stages in LDS at a time (multiple of 4)
  int32_t fpipe;  // the flush kernel keeps two whole windows in LDS (stages the next item's early)
  int32_t fw;     // the flush kernel forms the window weights and total decay itself (prep leaves them)
  float dt_min;
  // gated stale readout (no cold term for a skipped head): every head (hot_only), or the
  // heads whose query puts less than qgate_tau of its energy on the cold columns;
  // qcounts[0] / [1] (NULL: not counted) accumulate gated heads / heads that kept the term
  int32_t hot_only;
  float qgate_tau;
  unsigned long long* qcounts;
  // lagged teacher-forced readout (scale/nemo9b_eval.py:44,59,70, lag = 1): the read copy of
  // the snapshot before the last (cold2, scale2: cold's and scale's dtype and layout) and,
  // per (slot, head), the log-decay between those two snapshots (wlag)
  int32_t lag;
  void* cold2;
  float* scale2;
  float* wlag;
};

// Workspace carve-up for b requests (floats): rotated B and C [b][G][N] each,
// per-head scalars [b][H][HD_STRIDE]; tiered steps (c > 0) add the per-(request,
// group) flush flags [b][G] (int32, padded to a multiple of 4), window weights
// [b][H][c] (a flush whose weights prep forms) and the exact readout's window dots
// s_j = C'_cold . B'_j [b][G][c].
// HD_SNAPF is the factor of the snapshot readout: exp(glog) (stale, the decay up
// to the previous token), exp(glog + a) (exact, and teacher-forced between flushes:
// inclusive of this token), 1 (teacher-forced at a flush: the readout of the new state)
// or 0 (a head whose cold term the gated readout drops; HD_SKIP = 1 then).
enum { HD_DT = 0, HD_A, HD_DECAY, HD_SNAPF, HD_D, HD_FLUSH, HD_DTOT, HD_M, HD_POS, HD_SKIP, HD_AH, HD_STRIDE = 12 };
__host__ __device__ constexpr size_t flag_words(int b, int G, int c) {
  return c > 0 ? (((size_t)b * G + 3) & ~(size_t)3) : 0;
}
struct Ws {
  float *B, *C, *hd, *w, *s;
  int* fg;
  __host__ __device__ Ws(float* base, int b, int H, int G, int c) {
    B = base;
    C = B + (size_t)b * G * kN;
    hd = C + (size_t)b * G * kN;
    fg = reinterpret_cast<int*>(hd + (size_t)b * H * HD_STRIDE);
    w = hd + (size_t)b * H * HD_STRIDE + flag_words(b, G, c);
    s = w + (size_t)b * H * c;
  }
};
size_t ws_floats(int b, int H, int G, int c) {
  return (size_t)b * (2 * G * kN + H * HD_STRIDE + H * c + G * c) + flag_words(b, G, c);
}

__device__ __forceinline__ float bf2f(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// DPP controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror (lane i <-> 7-i within 8) = 0x141.
__device__ __forceinline__ float sum8(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v;
}
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  return v;
}

__device__ __forceinline__ float softplus_f(float v) { return v > 20.f ? v : log1pf(expf(v)); }

// Workgroup order of the unit kernel, whose logical order is (request, group, the group's W
// workgroups). The dispatcher deals workgroup i to XCD i % 8; in the paired order logical
// (request, group) pair 8m + x goes to XCD x, its W workgroups in a row, so the arrays a
// workgroup touches in less than whole cache lines (e4m3 row scales, y) and a pair's
// coefficient rows stay in one XCD's L2, while the eight XCDs still work on one compact
// window of the state (pairs 8m .. 8m + 7). Identity when the pair count is not a multiple
// of 8. Bit masks of the cold kinds that use it always (NSSM_COLD_FP8, _BF16_SINGLE,
// _FP8_BF16M) and of those that use it when the flush kernel does the flush (NSSM_COLD_FP32,
// _BF16), measured on MI355X in ms per 27-layer step: e4m3 over a bf16 master B=448 c=4
// 10.82 -> 10.59, ragged c=16 8.99 -> 8.82; e4m3 over an fp32 master 12.78 -> 12.68; single
// bf16 copy B=256 c=32 6.13 -> 6.04, c=4 6.16 -> 6.14; fp32 c=64 7.91 -> 7.86, c=32 7.97 ->
// 7.92, ragged B=384 c=64 12.18 -> 12.07, exact readout c=64 11.11 -> 10.58; bf16 read copy
// over an fp32 master c=64 6.09 -> 5.99. Where the stream kernel replays the window itself,
// fp32 cold (c=4 8.61 -> 8.69, its flush token slower; exact readout c=4 neutral, c=16 -1%)
// and the bf16 read copy (c=4 8.44 -> 8.50) keep the plain order, as does fresh_kernel
// (11.44 -> 11.46).
#ifndef NSSM_XCD_KINDS
#define NSSM_XCD_KINDS ((1 << NSSM_COLD_FP8) | (1 << NSSM_COLD_BF16_SINGLE) | (1 << NSSM_COLD_FP8_BF16M))
#endif
#ifndef NSSM_XCD_SPLIT_KINDS
#define NSSM_XCD_SPLIT_KINDS ((1 << NSSM_COLD_FP32) | (1 << NSSM_COLD_BF16))
#endif
__device__ __forceinline__ int xcd_order(int i, int W, int npairs) {
  if (npairs & 7) return i;
  const int k = i >> 3;
  return ((k / W) * 8 + (i & 7)) * W + k % W;
}

// Streaming access to the state: non-temporal (the state is touched once per
// token and is far larger than L2 and the MALL) unless built otherwise.
#ifndef NSSM_NT_LOAD
#define NSSM_NT_LOAD 1
#endif
#ifndef NSSM_NT_STORE
#define NSSM_NT_STORE 1
#endif
template <class T>
__device__ __forceinline__ T ld_stream(const T* p) {
  if constexpr (NSSM_NT_LOAD) return __builtin_nontemporal_load(p);
  else return *p;
}
template <class T>
__device__ __forceinline__ void st_stream(T v, T* p) {
  if constexpr (NSSM_NT_STORE) __builtin_nontemporal_store(v, p);
  else *p = v;
}
// The 16-bit arrays (the bf16 read copies and the bf16 master) are kept unit-blocked: the
// 8 rows of a unit (rows 8u .. 8u+7 of the [slots][H][P] row order) are one block of 8 NC
// elements, segment-major ([segment][8 rows][segment width]), so one wave instruction over
// a segment of a unit moves 512 contiguous bytes (whole cache lines) instead of 64 bytes of
// each of 8 rows. Segment s covers columns 32 s .. 32 s + w - 1 with w = min(32, NC - 32 s):
// every segment is 32 columns wide except a trailing 16-column one when NC % 32 == 16
// (k_hot = 16). Element (row, col) of such an array sits at blk16(row, col, NC); NC is a
// multiple of 16.
__host__ __device__ constexpr size_t blk16(size_t row, int col, int NC) {
  return (row >> 3) * (size_t)(8 * NC) + (size_t)(col >> 5) * 256 +
         (row & 7) * (size_t)(NC - (col & ~31) < 32 ? NC - (col & ~31) : 32) + (size_t)(col & 31);
}
constexpr int kBlkSeg = 64;  // u2v (4 bf16) between consecutive segments of a blocked row
// Offset of x ring element (sh = slot H + head, ring position pos, headdim row p), in the
// call's layout (StepArgs::xs_tok, xs_unit); rows p & ~7 .. p | 7 are contiguous.
__device__ __forceinline__ size_t xring(const StepArgs& a, size_t sh, int pos, int p) {
  return sh * (size_t)a.c * (size_t)a.P + (size_t)pos * (size_t)a.xs_tok + (size_t)(p >> 3) * (size_t)a.xs_unit +
         (size_t)(p & 7);
}

// ---------------------------------------------------------------------------
// prep: one workgroup (kPrepThreads threads) per (group g, block of prb <= kPrepReq requests).
//  * rotation: [B' C'] = R_g [B C] for the block, a 128 x 128 by 128 x 2 kPrepReq product
//    on the matrix cores (v_mfma_f32_16x16x4_f32, fp32 products and sums) in 16-column
//    tiles: columns j < kPrepReq are B of request j, the others C of request j - kPrepReq
//    (staged in LDS); wave w of W owns the output row tiles w, w + W, ... A lane loads R as
//    float4 (R[m][k..k+3]); the four MFMA steps of a 16-wide k block take the float4's
//    elements in turn, and the B operand takes the same k order, so each step pairs equal
//    k. The group's R is read once per block;
//  * one thread per (request, head) of the block computes the head's dt, decay,
//    stale-read factor, flush flag and, at a flush, the window weights; updates t,
//    nv, glog; appends dt and (rotation lanes) the B' cold columns to the ring at
//    position t % c. A flush token sits at c-1, so a flush window is always ring
//    positions [c-m, c).
// Latency bound: every independent global load is issued before the first barrier.
// Threads per prep workgroup: 8 waves, one rotation row tile each (at the 9B shape, 256
// threads (two row tiles per wave) measured 8.57 -> 8.14 us per launch at B = 256, c = 4,
// 11.65 -> 10.79 for the ragged B = 384, c = 64 batch and 15.5 -> 15.05 with the exact
// readout's window dots at c = 64: twice the loads in flight per CU).
#ifndef NSSM_PREP_THREADS
#define NSSM_PREP_THREADS 512
#endif
constexpr int kPrepThreads = NSSM_PREP_THREADS;
constexpr int kPrepRowTiles = (kN / 16) / (kPrepThreads / 64);  // rotation row tiles per wave
// Requests per prep workgroup (at most; a multiple of 8). Measured with 16 (a 128 x 32 product,
// half the workgroups): prep at the 9B shape 9.6 -> 12.9 us per launch at B = 256 and 13.5 ->
// 14.6 us at B = 384 (each workgroup's chain grows more than the launch shrinks).
constexpr int kPrepReq = 8;
constexpr int kPrepStage = kPrepReq * kN / kPrepThreads;  // B (and C) elements a prep thread stages
#ifndef NSSM_PREP_DOT_BATCH
#define NSSM_PREP_DOT_BATCH 4
#endif
constexpr int kPrepDotBatch = NSSM_PREP_DOT_BATCH;  // exact readout: window dots a prep lane group loads at once

// A head's dt (softplus, with the dt_min floor of the native path) and the scalars every
// stream kernel reads: dt, a = dt A, exp(a), D, A. Returns dt.
__device__ __forceinline__ float head_scalars(float* __restrict__ hd, float draw, float dtb, float Ah, float Dh,
                                              float dt_min) {
  float dt = softplus_f(draw + dtb);
  if (dt_min > 0.f) dt = fmaxf(dt, dt_min);
  const float av = dt * Ah;
  hd[HD_DT] = dt;
  hd[HD_A] = av;
  hd[HD_DECAY] = expf(av);
  hd[HD_D] = Dh;
  hd[HD_AH] = Ah;
  return dt;
}

// A pair flag naming the request's slot and its heads' window length m (1 <= m <= kMaxC < 128):
// positive, or -1 (the heads' scalars are read instead) for a slot past 2^24.
__device__ __forceinline__ int flush_flag(int slot, int m) { return slot < (1 << 24) ? (slot << 7) | m : -1; }

template <bool TIERED>
__global__ void __launch_bounds__(kPrepThreads) prep_kernel(StepArgs a) {
  __shared__ float sX[2 * kPrepReq][kN];  // B (j < kPrepReq) and C (j >= kPrepReq) of the block's requests
  __shared__ int sSlot[kPrepReq], sTr[kPrepReq], sNvr[kPrepReq];
  // per request of the block: its flushing heads in group g, and the least and greatest
  // window length among them (the pair flag, step 4)
  __shared__ int sFl[kPrepReq], sFmx[kPrepReq], sFmn[kPrepReq];
  // exact readout and query gate: B', C' of the block; each request's cold energy
  // fraction; gated / kept head counts
  __shared__ float sRot[TIERED ? 2 * kPrepReq : 1][TIERED ? kN : 1];
  __shared__ float sRho[kPrepReq];
  __shared__ int sQc[2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lk = lane >> 4;
  const int G = a.G, H = a.H, HG = a.HG, c = a.c;
  const int g = blockIdx.x % G, r0 = (blockIdx.x / G) * a.prb;
  const int nreq = min(a.prb, a.b - r0);
  const Ws ws(a.ws, a.b, H, G, c);
  const bool gate = TIERED && a.qgate_tau > 0.f && !a.hot_only;  // query gate (uniform)
  const bool rot_lds = TIERED && (a.exact || gate);              // B', C' kept in LDS

  if constexpr (!TIERED) {
    if (!a.R) {
      // untiered without a rotation: B and C converted straight into the workspace and the
      // head scalars written from registers, with no LDS and no barrier (at the 9B shape,
      // B = 256: 6.2 us per launch through the staged path). Every load is issued before
      // the first store (one memory round trip, not one per element a thread converts).
      // (a thread's elements past the block load its last element, so no load is predicated)
      float bv[kPrepStage], cv[kPrepStage];
#pragma unroll
      for (int u = 0; u < kPrepStage; ++u) {
        const int i = min(tid + u * kPrepThreads, nreq * kN - 1);
        const size_t o = ((size_t)r0 * G + g) * kN + (size_t)(i / kN) * G * kN + (i % kN);
        bv[u] = bf2f(a.Bm[o]);
        cv[u] = bf2f(a.Cm[o]);
      }
#pragma unroll
      for (int u = 0; u < kPrepStage; ++u) {
        const int i = tid + u * kPrepThreads;
        const size_t o = ((size_t)r0 * G + g) * kN + (size_t)(i / kN) * G * kN + (i % kN);
        if (i < nreq * kN) {
          ws.B[o] = bv[u];
          ws.C[o] = cv[u];
        }
      }
      if (tid < nreq * HG) {
        const int hr = tid / HG, h = g * HG + (tid - hr * HG), bi = r0 + hr;
        const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
        if (slot >= 0 && slot < a.slots) {
          float* __restrict__ hd = ws.hd + ((size_t)bi * H + h) * HD_STRIDE;
          head_scalars(hd, bf2f(a.dt_raw[(size_t)bi * H + h]), a.dt_bias[h], a.A[h], a.D[h], a.dt_min);
          hd[HD_SNAPF] = 0.f;
          hd[HD_FLUSH] = 0.f;
          hd[HD_DTOT] = 1.f;
          hd[HD_M] = 0.f;
          hd[HD_POS] = 0.f;
        }
      }
      return;
    }
  }

  // 1. independent loads: B and C of the block (zero past the last request), R, the
  // head inputs, all issued before the first LDS store
  // (rows past the block load the block's last request and are zeroed after, so no load is
  // predicated)
  float bst[kPrepStage], cst[kPrepStage];
#pragma unroll
  for (int u = 0; u < kPrepStage; ++u) {
    const int i = tid + u * kPrepThreads, r = i / kN, n = i - r * kN;
    const size_t o = ((size_t)(r0 + min(r, nreq - 1)) * G + g) * kN + n;
    bst[u] = bf2f(a.Bm[o]);
    cst[u] = bf2f(a.Cm[o]);
    if (r >= nreq) bst[u] = cst[u] = 0.f;
  }
  const float* __restrict__ Rg = a.R ? a.R + (size_t)g * kN * kN : nullptr;
  f4 ra[kPrepRowTiles][kN / 16];  // this lane's R operands of its row tiles
  if (Rg) {
#pragma unroll
    for (int t2 = 0; t2 < kPrepRowTiles; ++t2)
#pragma unroll
      for (int kb = 0; kb < kN / 16; ++kb)
        ra[t2][kb] = *reinterpret_cast<const f4*>(
            Rg + (size_t)((wave + (kPrepThreads / 64) * t2) * 16 + li) * kN + kb * 16 + 4 * lk);
  }
  if (tid < kPrepReq) {
    sFl[tid] = 0;
    sFmx[tid] = 0;
    sFmn[tid] = kMaxC + 1;
  }
  if (tid < 2) sQc[tid] = 0;
  const int hr = tid / HG, hh = tid - hr * HG;  // the head thread's request and head
  const bool head_thread = tid < nreq * HG;
  const int h = g * HG + hh, bi = r0 + hr;
  int slot = -1, tt = 0, nvv = 0;
  float draw = 0.f, dtb = 0.f, Ah = 0.f, Dh = 0.f, gl = 0.f;
  if (head_thread) {
    slot = a.slot_ids ? a.slot_ids[bi] : bi;
    draw = bf2f(a.dt_raw[(size_t)bi * H + h]);
    dtb = a.dt_bias[h];
    Ah = a.A[h];
    Dh = a.D[h];
    if constexpr (TIERED) {
      // t >= 0 and 0 <= nv <= t % c hold for every tier these kernels write (a join
      // sets nv = 0 at any phase, each token then advances both, a flush zeroes nv);
      // the clamps keep every ring offset (t % c - nv + j, c - 1 - nv) in [0, c) even
      // for a tier whose t or nv was written by hand
      if (slot >= 0 && slot < a.slots) {
        const size_t o = (size_t)slot * H + h;
        tt = max(a.t[o], 0);
        nvv = min(max(a.nv[o], 0), tt % c);
        gl = a.glog[o];
      }
    }
    if (hh == 0) {
      sSlot[hr] = slot;
      sTr[hr] = tt;
      sNvr[hr] = nvv;
    }
  }
#pragma unroll
  for (int u = 0; u < kPrepStage; ++u) {
    const int i = tid + u * kPrepThreads, r = i / kN, n = i - r * kN;
    sX[r][n] = bst[u];
    sX[kPrepReq + r][n] = cst[u];
  }
  __syncthreads();

  // 2. rotation and its stores: column tile ct of the product holds columns j = 16 ct + li
  // (B of request j for j < kPrepReq, C of request j - kPrepReq after)
  if (Rg) {
#pragma unroll
    for (int t2 = 0; t2 < kPrepRowTiles; ++t2) {
#pragma unroll
      for (int ct = 0; ct < 2 * kPrepReq / 16; ++ct) {
        f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < kN / 16; ++kb) {
          const f4 xb = *reinterpret_cast<const f4*>(&sX[16 * ct + li][kb * 16 + 4 * lk]);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[t2][kb].x, xb.x, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[t2][kb].y, xb.y, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[t2][kb].z, xb.z, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[t2][kb].w, xb.w, acc, 0, 0, 0);
        }
        // lane (li, lk) holds rows m0 + 4 lk .. +3 of column 16 ct + li
        const int m0 = (wave + (kPrepThreads / 64) * t2) * 16 + 4 * lk;
        const int j = 16 * ct + li, r = j % kPrepReq, which = j / kPrepReq;
        if constexpr (TIERED) {
          if (rot_lds) *reinterpret_cast<f4*>(&sRot[j][m0]) = acc;
        }
        const int sl = r < nreq ? sSlot[r] : -1;
        if (sl >= 0 && sl < a.slots) {
          *reinterpret_cast<f4*>((which ? ws.C : ws.B) + ((size_t)(r0 + r) * G + g) * kN + m0) = acc;
          if constexpr (TIERED) {
            // ring append of the B' cold columns (tokens that do not flush; a flush
            // token's columns are read from the workspace). x goes to the ring from
            // the stream kernel.
            const int tr = sTr[r];
            if (which == 0 && m0 >= a.K && (tr + 1) % c != 0)
              *reinterpret_cast<f4*>(a.ring_b + (((size_t)sl * G + g) * c + tr % c) * (kN - a.K) + (m0 - a.K)) = acc;
          }
        }
      }
    }
  } else {  // identity rotation
    for (int i = tid; i < nreq * kN; i += kPrepThreads) {
      const int r = i / kN, n = i - r * kN;
      const int sl = sSlot[r];
      if (sl < 0 || sl >= a.slots) continue;
      const size_t o = ((size_t)(r0 + r) * G + g) * kN + n;
      ws.B[o] = sX[r][n];
      ws.C[o] = sX[kPrepReq + r][n];
      if constexpr (TIERED) {
        if (rot_lds) {
          sRot[r][n] = sX[r][n];
          sRot[kPrepReq + r][n] = sX[kPrepReq + r][n];
        }
        const int tr = sTr[r];
        if (n >= a.K && (tr + 1) % c != 0)
          a.ring_b[(((size_t)sl * G + g) * c + tr % c) * (kN - a.K) + (n - a.K)] = sX[r][n];
      }
    }
  }

  // 2b. exact readout: s_j = C'_cold . B'_j for each request's window, j = 0 .. nv
  // (buffered tokens at ring positions t % c - nv + j, then this token), written to the
  // workspace per (request, group); the stream kernel forms the weights w_j and sums
  // w_j s_j x_j itself. (Splitting the buffered positions over four workgroups per (group,
  // request block), each repeating the rotation, measured slower: 15.0 -> 18.7 us per
  // launch at the 9B shape, B = 256, c = 64.)
  if constexpr (TIERED) {
    if (a.exact) {
      __syncthreads();  // sRot
      // 8 lanes per (request, window token): lane k of the group takes columns K + 32 i + 4 k
      // (float4 each), then a DPP sum over the group's 8 lanes. The loop bounds are uniform
      // over each aligned 8-lane group, so every group's lanes sum together.
      const int NC = kN - a.K, k8 = tid & 7;
      float* __restrict__ sw = ws.s + ((size_t)r0 * G + g) * c;  // request r: sw + r G c
      constexpr int NG = kPrepThreads / 8;  // 8-lane groups
      // buffered positions of the block's longest live window, j = 0 .. nb - 1 (at the 9B
      // shape, B = 256, c = 64: 23.1 -> 22.0 us per launch on average, 14.8 -> 9.3 with one
      // token buffered, against items over all c positions)
      int nb = 0;
      for (int r = 0; r < nreq; ++r) nb = max(nb, sNvr[r]);
      const int ni = nreq * nb, nc = nreq;  // buffered items, this token's items
      if (ni + nc <= NG) {
        // one item per group: buffered tokens from the ring, then this token from LDS
        const int it = tid >> 3;
        if (it < ni + nc) {
          const bool cur = it >= ni;
          const int r = cur ? it - ni : it / nb, j = cur ? sNvr[r] : it - r * nb;
          const int sl2 = sSlot[r], nv = sNvr[r];
          const bool live = sl2 >= 0 && sl2 < a.slots && (cur || j < nv);
          float acc = 0.f;
          if (live) {
            const float* bj = cur ? &sRot[r][a.K] : a.ring_b + (((size_t)sl2 * G + g) * c + (sTr[r] % c - nv + j)) * NC;
            const float* cq = &sRot[kPrepReq + r][a.K];
            f4 bv[kN / 32], cv[kN / 32];
#pragma unroll
            for (int i = 0; i < kN / 32; ++i) {  // NC is a multiple of 16: a float4 is inside or past it
              if (32 * i + 4 * k8 < NC) {
                bv[i] = *reinterpret_cast<const f4*>(bj + 32 * i + 4 * k8);
                cv[i] = *reinterpret_cast<const f4*>(cq + 32 * i + 4 * k8);
              }
            }
#pragma unroll
            for (int i = 0; i < kN / 32; ++i) {
              if (32 * i + 4 * k8 < NC) {
                acc = fmaf(bv[i].x, cv[i].x, acc);
                acc = fmaf(bv[i].y, cv[i].y, acc);
                acc = fmaf(bv[i].z, cv[i].z, acc);
                acc = fmaf(bv[i].w, cv[i].w, acc);
              }
            }
          }
          acc = sum8(acc);
          if (live && k8 == 0) sw[(size_t)r * G * c + j] = acc;
        }
      } else {
        // more items than groups: buffered tokens from the ring, kPrepDotBatch items per
        // group and round with every load unpredicated (an item that is not buffered, or of
        // a slot out of range, reads its request's first buffered row, which live items read
        // too; a column past the cold tier reads the tier's last float4; both dropped), so
        // each round is one memory round trip; then this token from LDS
        for (int it0 = tid >> 3; it0 < ni; it0 += kPrepDotBatch * NG) {
          f4 bv[kPrepDotBatch][kN / 32];
#pragma unroll
          for (int u = 0; u < kPrepDotBatch; ++u) {
            const int it = min(it0 + u * NG, ni - 1), r = it / nb, j = it - r * nb;
            const int sl2 = sSlot[r], nv = sNvr[r];
            const int slc = sl2 >= 0 && sl2 < a.slots ? sl2 : 0;
            const int pos = sTr[r] % c - nv + (j < nv ? j : 0);  // in [0, c): nv <= t % c
            const float* bj = a.ring_b + (((size_t)slc * G + g) * c + pos) * NC;
#pragma unroll
            for (int i = 0; i < kN / 32; ++i)
              bv[u][i] = *reinterpret_cast<const f4*>(bj + min(32 * i + 4 * k8, NC - 4));
          }
#pragma unroll
          for (int u = 0; u < kPrepDotBatch; ++u) {
            const int itr = it0 + u * NG, it = min(itr, ni - 1), r = it / nb, j = it - r * nb;
            const int sl2 = sSlot[r];
            const bool live = itr < ni && sl2 >= 0 && sl2 < a.slots && j < sNvr[r];
            const float* cq = &sRot[kPrepReq + r][a.K];
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < kN / 32; ++i) {
              if (32 * i + 4 * k8 < NC) {
                const f4 cv = *reinterpret_cast<const f4*>(cq + 32 * i + 4 * k8);
                acc = fmaf(bv[u][i].x, cv.x, acc);
                acc = fmaf(bv[u][i].y, cv.y, acc);
                acc = fmaf(bv[u][i].z, cv.z, acc);
                acc = fmaf(bv[u][i].w, cv.w, acc);
              }
            }
            acc = sum8(acc);
            if (live && k8 == 0) sw[(size_t)r * G * c + j] = acc;
          }
        }
        for (int r = tid >> 3; r < nc; r += NG) {
          const int sl2 = sSlot[r];
          const float* bq = &sRot[r][a.K];
          const float* cq = &sRot[kPrepReq + r][a.K];
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < kN / 32; ++i) {
            if (32 * i + 4 * k8 < NC) {
              const f4 b4 = *reinterpret_cast<const f4*>(bq + 32 * i + 4 * k8);
              const f4 c4 = *reinterpret_cast<const f4*>(cq + 32 * i + 4 * k8);
              acc = fmaf(b4.x, c4.x, acc);
              acc = fmaf(b4.y, c4.y, acc);
              acc = fmaf(b4.z, c4.z, acc);
              acc = fmaf(b4.w, c4.w, acc);
            }
          }
          acc = sum8(acc);
          if (sl2 >= 0 && sl2 < a.slots && k8 == 0) sw[(size_t)r * G * c + sNvr[r]] = acc;
        }
      }
    }
  }

  // 2c. query gate: rho_r = sum_{n>=K} C'_n^2 / max(sum_n C'_n^2, 1e-9) of each request
  // (scale/v4_native_decode.py:147-156); 8 lanes per request
  if constexpr (TIERED) {
    if (gate) {
      __syncthreads();  // sRot
      if (tid < 8 * kPrepReq) {
        const int r = tid >> 3, j = tid & 7;
        float ea = 0.f, ec = 0.f;
        for (int n = 4 * j; n < kN; n += 32) {  // K is a multiple of 16: a float4 is hot or cold
          const f4 v = *reinterpret_cast<const f4*>(&sRot[kPrepReq + r][n]);
          const float e = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
          ea += e;
          if (n >= a.K) ec += e;
        }
        ea = sum8(ea);
        ec = sum8(ec);
        // clamp(min=1e-9) keeps a NaN energy NaN, so its head is dropped
        if (j == 0) sRho[r] = ec / (ea < 1e-9f ? 1e-9f : ea);
      }
      __syncthreads();  // sRho
    }
  }

  // 3. per-head scalars and bookkeeping
  if (head_thread && slot >= 0 && slot < a.slots) {
    float* __restrict__ hd = ws.hd + ((size_t)bi * H + h) * HD_STRIDE;
    const float dt = head_scalars(hd, draw, dtb, Ah, Dh, a.dt_min), av = dt * Ah;
    if constexpr (TIERED) {
      const size_t o = (size_t)slot * H + h;
      const int pos = tt % c;
      const bool flush = (tt + 1) % c == 0;  // then pos == c - 1
      const bool exact = a.exact != 0;
      // gated readout: coldoff drops every head's cold term (scale/v4_native_decode.py:118-127),
      // the query gate a head whose rho < tau (:147-156); the tier evolves as without it
      bool skip = !exact && a.hot_only;
      if (gate) {
        const bool keep = sRho[hr] >= a.qgate_tau;
        skip = !keep;
        if (a.qcounts) {
          atomicAdd(&sQc[0], 1);
          if (keep) atomicAdd(&sQc[1], 1);
        }
      }
      // stale: exp(glog), the decay up to the previous token (one-token lag);
      // exact: exp(glog + a), inclusive of this token (scale/v4_native_decode.py:89)
      // teacher-forced (scale/nemo9b_eval.py:57-70): the snapshot is the state after the flush
      // token's update, read undecayed at that token and with inclusive decay after it;
      // lagged (:59,70): the snapshot before it, decayed by the window between the two (wlag)
      // as well; at a flush the old snapshot becomes the lagged one, wlag this window's decay
      if (a.lag) {
        const float wl = a.wlag[o];
        hd[HD_SNAPF] = expf(flush ? gl + av : gl + av + wl);
        if (flush) a.wlag[o] = gl + av;
      } else {
        hd[HD_SNAPF] = skip ? 0.f : a.tf ? (flush ? 1.f : expf(gl + av)) : expf(exact ? gl + av : gl);
      }
      hd[HD_SKIP] = skip ? 1.f : 0.f;
      hd[HD_FLUSH] = flush ? 1.f : 0.f;
      hd[HD_POS] = (float)pos;
      if (flush) {
        atomicAdd(&sFl[hr], 1);
        atomicMax(&sFmx[hr], nvv + 1);
        atomicMin(&sFmn[hr], nvv + 1);
      }
      if (flush && !a.fw) {
        // window = the nv buffered tokens at ring [pos-nv, pos) and this one (at a
        // flush pos = c-1): w_i = exp(sum_{l>i} a_l) dt_i, total decay exp(sum_l a_l).
        // The buffered dt are loaded 16 at a time.
        const int mw = nvv + 1;
        const float* __restrict__ rdt = a.ring_dt + o * c + (pos - nvv);
        float* __restrict__ w = ws.w + ((size_t)bi * H + h) * c;
        w[mw - 1] = dt;
        float suf = dt * Ah;
        for (int i0 = mw - 2; i0 >= 0; i0 -= 16) {
          float v[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) v[u] = i0 - u >= 0 ? rdt[i0 - u] : 0.f;
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            if (i0 - u >= 0) {
              w[i0 - u] = expf(suf) * v[u];
              suf += v[u] * Ah;
            }
          }
        }
        hd[HD_DTOT] = expf(suf);
        hd[HD_M] = (float)mw;
      } else {
        // the flush kernel forms a flushing window's weights from the ring's dt, the exact
        // readout's stream kernel its correction weights; both read the window length
        hd[HD_DTOT] = 1.f;
        hd[HD_M] = flush || exact ? (float)(nvv + 1) : 0.f;
      }
      if (flush) {
        a.nv[o] = 0;
        a.glog[o] = 0.f;
      } else {
        a.ring_dt[o * c + pos] = dt;
        a.nv[o] = nvv + 1;
        a.glog[o] = gl + av;
      }
      a.t[o] = tt + 1;
    } else {
      hd[HD_SNAPF] = 0.f;
      hd[HD_FLUSH] = 0.f;
      hd[HD_DTOT] = 1.f;
      hd[HD_M] = 0.f;
      hd[HD_POS] = 0.f;
    }
  }
  // 4. the flush kernel's per-(request, group) flags (every pair of the block is written, so
  // no flag survives from an earlier token): 0, no head of the pair flushes; otherwise
  // flush_flag of the request's slot and window length when every head of the pair flushes
  // a window of the same length (the flush kernel then lists the pair's heads without
  // reading their scalars), else -1
  if constexpr (TIERED) {
    if (a.split || (gate && a.qcounts)) {
      __syncthreads();
      if (a.split && tid < nreq) {
        const int n = sFl[tid];
        ws.fg[(size_t)(r0 + tid) * G + g] = n == 0 ? 0 : n == HG && sFmx[tid] == sFmn[tid] ? flush_flag(sSlot[tid], sFmx[tid]) : -1;
      }
      if (gate && a.qcounts && tid == 0) {
        atomicAdd(a.qcounts, (unsigned long long)sQc[0]);
        atomicAdd(a.qcounts + 1, (unsigned long long)sQc[1]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// stream kernel
//
// Lane mappings inside a unit (8 rows p0..p0+7 of one head); lane l, rr = l >> 3, q = l & 7:
//   segment     columns 32 s + 4 q + e of row p0 + rr (segment s, e = 0..3): hot columns, the
//               fp32 cold copy, the fp32 master (one dwordx4 per segment moves 8 rows x 128 B,
//               whole cache lines, per wave instruction), the bf16 read copies and the bf16
//               master (unit-blocked, one dwordx2 per segment: 512 contiguous bytes). A
//               16-column half segment (the hot tier and the tail of the cold one at
//               k_hot = 16) gives lane q columns 2 q, 2 q + 1 of it (one dwordx2 of fp32, one
//               dword of bf16: 8 rows x 64 B).
//   contiguous  columns CW q .. CW q + CW - 1 (CW = NC / 8) of row p0 + rr: the e4m3 read
//               copies, so a lane's bytes are one contiguous dwordx3 (k = 32) load. At
//               k_hot = 16 (CW = 14, lane parts not word aligned) e4m3 is read in the segment
//               mapping instead (a dword per segment, two bytes of the half segment).
//   mfma        flush at c >= 16: lane (li = l & 15, lk = l >> 4) of a 16 x 16 tile holds row
//               p0 + li, columns n0 + 4 lk .. +3: the accumulator layout of v_mfma_f32_16x16x4_f32.
// Both unit mappings group a row's lanes as 8 consecutive lanes, so a row's dot product is
// sum8 (three DPP steps).

// Cold storage kinds (include/nssm.h) by read copy and master:
//   kind            read copy (mapping)          master
//   FP32            fp32 (segment)               the read copy
//   BF16_SINGLE     bf16 (segment)               the read copy
//   BF16            bf16 (segment)               fp32
//   FP8             e4m3 + row scale (contig.)   fp32
//   FP8_BF16M       e4m3 + row scale (contig.)   bf16
// A single copy is read in the segment mapping so a flushing head replays onto the
// values it read; a master beside a read copy is loaded only by flushing heads. The 16-bit
// copies are unit-blocked (blk16); the e4m3 copies row-major, read contiguously.
template <int K, int COLD>
struct Cfg {
  static constexpr int HS = K / 32;                              // full hot segments
  static constexpr bool HH = (K % 32) != 0;                      // a hot half segment (K = 16)
  static constexpr int HSR = HS > 0 ? HS : 1;
  static constexpr int NC = kN - K;
  static constexpr bool TIERED = COLD != NSSM_COLD_NONE && NC > 0;
  static constexpr int CS = TIERED ? NC / 32 : 0;                // full cold segments per row
  static constexpr bool CH = TIERED && (NC % 32) != 0;           // a cold half segment (K = 16)
  static constexpr int CSR = CS > 0 ? CS : 1;
  static constexpr bool E4M3 = COLD == NSSM_COLD_FP8 || COLD == NSSM_COLD_FP8_BF16M;  // e4m3 read copy
  static constexpr bool SEG = COLD == NSSM_COLD_FP32 || COLD == NSSM_COLD_BF16_SINGLE;  // single copy
  static constexpr bool B16 = COLD == NSSM_COLD_BF16 || COLD == NSSM_COLD_BF16_SINGLE;  // bf16 read copy
  static constexpr bool CONTIG = E4M3 && !CH;                                           // contiguous e4m3 read
  static constexpr bool SEG8 = E4M3 && CH;                                              // segment e4m3 read
  static constexpr bool SEGREAD = SEG || B16 || SEG8;                                   // segment read
  static constexpr bool MASTER32 = COLD == NSSM_COLD_BF16 || COLD == NSSM_COLD_FP8;    // fp32 master
  static constexpr bool MASTER16 = COLD == NSSM_COLD_FP8_BF16M;                        // bf16 master
  static constexpr int CW = NC / 8;                              // contiguous columns per lane
  static constexpr int WORDS = CONTIG ? CW / 4 : 0;
  static constexpr int WR = WORDS > 0 ? WORDS : 1;
  static constexpr int CWR = CONTIG ? CW : 1;
  static constexpr int NT = NC / 16;                             // 16-column tiles of a row
};

typedef float f2 __attribute__((ext_vector_type(2)));

// e4m3fn <-> fp32 on gfx950's conversion instructions (OCP e4m3fn, round to nearest even;
// bit-identical to nssm_f32_to_e4m3fn / nssm_e4m3fn_to_f32 for the |v| <= 448 range the
// kernels produce)
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float (&v)[4]) {
  const f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  v[0] = lo.x; v[1] = lo.y; v[2] = hi.x; v[3] = hi.y;
}
__device__ __forceinline__ uint32_t f32x4_to_fp8(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

template <int N>
__device__ __forceinline__ void ld_words(const uint32_t* p, uint32_t (&w)[N]) {
  if constexpr (N == 1) {
    w[0] = ld_stream(p);
  } else if constexpr (N == 2) {
    const u2v t = ld_stream(reinterpret_cast<const u2v*>(p));
    w[0] = t.x; w[1] = t.y;
  } else if constexpr (N == 3) {  // 12 bytes at 4-byte alignment
    w[0] = ld_stream(p);
    w[1] = ld_stream(p + 1);
    w[2] = ld_stream(p + 2);
  } else {
    static_assert(N % 2 == 0, "word count");
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      const u2v t = ld_stream(reinterpret_cast<const u2v*>(p + i));
      w[i] = t.x; w[i + 1] = t.y;
    }
  }
}

// Raw registers of one unit for one lane.
template <int K, int COLD>
struct UnitRaw {
  using C = Cfg<K, COLD>;
  f4 hv[C::HSR];
  f2 hh;                                                     // hot half segment
  f4 cf[COLD == NSSM_COLD_FP32 ? C::CSR : 1];               // fp32 cold copy, segment mapping
  f2 cfh;                                                    // ... its half segment
  u2v cb[C::B16 ? C::CSR : 1];                              // bf16 read copy, segment mapping
  uint32_t cbh;                                              // ... its half segment (2 x bf16)
  uint32_t cw[C::WR];                                        // e4m3 read copy, contiguous mapping
  uint32_t c8[C::SEG8 ? C::CSR : 1];                        // e4m3 read copy, segment mapping
  uint32_t c8h;                                              // ... its half segment (2 bytes)
  float sc;                                     // e4m3 row scale
  float xp;
  uint16_t xraw;
};

// The rotated coefficients a lane needs for its columns: B', C' of the hot columns and C' of
// the cold ones, in the mappings the unit reads its state in.
template <int K, int COLD>
struct Coef {
  using C = Cfg<K, COLD>;
  float Bh[C::HSR][4], Ch[C::HSR][4];  // hot segments
  float Bhh[2], Chh[2];                // hot half segment
  float Cc[C::CSR][4], Cch[2];         // cold segments (segment reads) and the cold half segment
  float Cq[C::CWR];                    // cold columns of the contiguous e4m3 mapping
};

// SEGC: also the cold columns' C' in the segment mapping (the segment reads, and the
// teacher-forced flush readout of the values the lane stores)
template <int K, int COLD, bool SEGC = Cfg<K, COLD>::SEGREAD>
__device__ __forceinline__ void coef_load(const float* wB, const float* wC, int q, Coef<K, COLD>& k) {
  using C = Cfg<K, COLD>;
#pragma unroll
  for (int s = 0; s < C::HS; ++s) {
    const f4 tb = *reinterpret_cast<const f4*>(wB + 32 * s + 4 * q);
    const f4 tc = *reinterpret_cast<const f4*>(wC + 32 * s + 4 * q);
    k.Bh[s][0] = tb.x; k.Bh[s][1] = tb.y; k.Bh[s][2] = tb.z; k.Bh[s][3] = tb.w;
    k.Ch[s][0] = tc.x; k.Ch[s][1] = tc.y; k.Ch[s][2] = tc.z; k.Ch[s][3] = tc.w;
  }
  if constexpr (C::HH) {
    const f2 tb = *reinterpret_cast<const f2*>(wB + 32 * C::HS + 2 * q);
    const f2 tc = *reinterpret_cast<const f2*>(wC + 32 * C::HS + 2 * q);
    k.Bhh[0] = tb.x; k.Bhh[1] = tb.y;
    k.Chh[0] = tc.x; k.Chh[1] = tc.y;
  }
#pragma unroll
  for (int s = 0; s < C::CSR; ++s) {
    if constexpr (SEGC && C::CS > 0) {
      const f4 tc = *reinterpret_cast<const f4*>(wC + K + 32 * s + 4 * q);
      k.Cc[s][0] = tc.x; k.Cc[s][1] = tc.y; k.Cc[s][2] = tc.z; k.Cc[s][3] = tc.w;
    } else {
      k.Cc[s][0] = k.Cc[s][1] = k.Cc[s][2] = k.Cc[s][3] = 0.f;
    }
  }
  if constexpr (C::CH) {
    const f2 tc = *reinterpret_cast<const f2*>(wC + K + 32 * C::CS + 2 * q);
    k.Cch[0] = tc.x; k.Cch[1] = tc.y;
  }
#pragma unroll
  for (int i = 0; i < C::CWR; ++i) {
    if constexpr (C::CONTIG) k.Cq[i] = wC[K + C::CW * q + i];
    else k.Cq[i] = 0.f;
  }
}

// cold_src / scale_src: the read copy to read (default the tier's; the lagged readout reads
// its second one)
template <int K, int COLD>
__device__ __forceinline__ void unit_load(const StepArgs& a, size_t row, size_t xrow, int q, UnitRaw<K, COLD>& d,
                                          bool hot_only = false, const void* cold_src = nullptr,
                                          const float* scale_src = nullptr) {
  using C = Cfg<K, COLD>;
  const void* const cold = cold_src ? cold_src : a.cold;
  const float* const scale = scale_src ? scale_src : a.scale;
  const f4* hp = reinterpret_cast<const f4*>(a.hot + row * K) + q;
#pragma unroll
  for (int s = 0; s < C::HS; ++s) d.hv[s] = ld_stream(hp + 8 * s);
  if constexpr (C::HH) d.hh = ld_stream(reinterpret_cast<const f2*>(a.hot + row * K + 32 * C::HS) + q);
  if constexpr (C::TIERED) {
    if (!hot_only) {
      if constexpr (COLD == NSSM_COLD_FP32) {
        const float* rp = static_cast<const float*>(cold) + row * C::NC;
        const f4* p = reinterpret_cast<const f4*>(rp) + q;
#pragma unroll
        for (int s = 0; s < C::CS; ++s) d.cf[s] = ld_stream(p + 8 * s);
        if constexpr (C::CH) d.cfh = ld_stream(reinterpret_cast<const f2*>(rp + 32 * C::CS) + q);
      } else if constexpr (C::B16) {
        const uint16_t* base = static_cast<const uint16_t*>(cold);
        const u2v* p = reinterpret_cast<const u2v*>(base + blk16(row, 4 * q, C::NC));
#pragma unroll
        for (int s = 0; s < C::CS; ++s) d.cb[s] = ld_stream(p + kBlkSeg * s);
        if constexpr (C::CH)
          d.cbh = ld_stream(reinterpret_cast<const uint32_t*>(base + blk16(row, 32 * C::CS + 2 * q, C::NC)));
      } else if constexpr (C::SEG8) {
        const uint8_t* rp = static_cast<const uint8_t*>(cold) + row * C::NC;
        const uint32_t* p = reinterpret_cast<const uint32_t*>(rp) + q;
#pragma unroll
        for (int s = 0; s < C::CS; ++s) d.c8[s] = ld_stream(p + 8 * s);
        d.c8h = ld_stream(reinterpret_cast<const uint16_t*>(rp + 32 * C::CS) + q);
        d.sc = scale[row];
      } else {
        ld_words<C::WORDS>(
            reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(cold) + row * C::NC + C::CW * q), d.cw);
        d.sc = scale[row];
      }
    }
  }
  d.xraw = a.x[xrow];
  d.xp = bf2f(d.xraw);
}

// The lagged readout's flush: the old read copy as unit_load read it (d), written to the
// tier's second read copy in the same mapping, before the flush replaces the first.
template <int K, int COLD>
__device__ __forceinline__ void lag_store(const StepArgs& a, size_t row, int q, const UnitRaw<K, COLD>& d) {
  using C = Cfg<K, COLD>;
  if constexpr (C::TIERED) {
    if constexpr (COLD == NSSM_COLD_FP32) {
      float* rp = static_cast<float*>(a.cold2) + row * C::NC;
      f4* p = reinterpret_cast<f4*>(rp) + q;
#pragma unroll
      for (int s = 0; s < C::CS; ++s) st_stream(d.cf[s], p + 8 * s);
      if constexpr (C::CH) st_stream(d.cfh, reinterpret_cast<f2*>(rp + 32 * C::CS) + q);
    } else if constexpr (C::B16) {
      uint16_t* base = static_cast<uint16_t*>(a.cold2);
      u2v* p = reinterpret_cast<u2v*>(base + blk16(row, 4 * q, C::NC));
#pragma unroll
      for (int s = 0; s < C::CS; ++s) st_stream(d.cb[s], p + kBlkSeg * s);
      if constexpr (C::CH) st_stream(d.cbh, reinterpret_cast<uint32_t*>(base + blk16(row, 32 * C::CS + 2 * q, C::NC)));
    } else if constexpr (C::SEG8) {
      uint8_t* rp = static_cast<uint8_t*>(a.cold2) + row * C::NC;
      uint32_t* p = reinterpret_cast<uint32_t*>(rp) + q;
#pragma unroll
      for (int s = 0; s < C::CS; ++s) st_stream(d.c8[s], p + 8 * s);
      st_stream((uint16_t)d.c8h, reinterpret_cast<uint16_t*>(rp + 32 * C::CS) + q);
      if (q == 0) a.scale2[row] = d.sc;
    } else {
      uint32_t* p = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.cold2) + row * C::NC + C::CW * q);
#pragma unroll
      for (int i = 0; i < C::WORDS; ++i) st_stream(d.cw[i], p + i);
      if (q == 0) a.scale2[row] = d.sc;
    }
  }
}

__device__ __forceinline__ void bf16x4_to_f32(u2v w, float (&v)[4]) {
  v[0] = __uint_as_float(w.x << 16);
  v[1] = __uint_as_float(w.x & 0xffff0000u);
  v[2] = __uint_as_float(w.y << 16);
  v[3] = __uint_as_float(w.y & 0xffff0000u);
}
__device__ __forceinline__ void bf16x2_to_f32(uint32_t w, float (&v)[2]) {
  v[0] = __uint_as_float(w << 16);
  v[1] = __uint_as_float(w & 0xffff0000u);
}
// RNE to bf16 with gfx950's packed conversion (v_cvt_pk_bf16_f32), bit-identical to
// nssm_f32_to_bf16 for non-NaN values, subnormals and ties included (checked against
// torch's cast by the join test); 1-2% faster than the software rounding on the flush paths.
__device__ __forceinline__ uint32_t f32x2_to_bf16(float a, float b) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), b2));
}
__device__ __forceinline__ u2v f32x4_to_bf16(float a, float b, float c, float d) {
  return u2v{f32x2_to_bf16(a, b), f32x2_to_bf16(c, d)};
}

// w / sc rounded to nearest for sc > 0: one correctly rounded reciprocal per row, then
// q = w inv and one correction step q + (w - q sc) inv (Markstein: correctly rounded when
// inv is and no intermediate over- or underflows); the sign of w restores -0 (the
// correction step sums +0 and -0 to +0). Three operations per value instead of an IEEE
// division's sequence.
struct QDiv {
  float sc, inv;
  __device__ __forceinline__ explicit QDiv(float s) : sc(s), inv(1.0f / s) {}
  __device__ __forceinline__ float operator()(float w) const {
    const float q = w * inv;
    return copysignf(fmaf(fmaf(-q, sc, w), inv, q), w);
  }
};

// stale readout partial of one lane from its read-copy registers (times the row scale for e4m3)
template <int K, int COLD>
__device__ __forceinline__ float cold_partial(const UnitRaw<K, COLD>& d, const Coef<K, COLD>& k) {
  using C = Cfg<K, COLD>;
  float pc = 0.f;
  if constexpr (COLD == NSSM_COLD_FP32) {
#pragma unroll
    for (int s = 0; s < C::CS; ++s) {
      pc = fmaf(d.cf[s].x, k.Cc[s][0], pc);
      pc = fmaf(d.cf[s].y, k.Cc[s][1], pc);
      pc = fmaf(d.cf[s].z, k.Cc[s][2], pc);
      pc = fmaf(d.cf[s].w, k.Cc[s][3], pc);
    }
    if constexpr (C::CH) {
      pc = fmaf(d.cfh.x, k.Cch[0], pc);
      pc = fmaf(d.cfh.y, k.Cch[1], pc);
    }
  } else if constexpr (C::B16) {
#pragma unroll
    for (int s = 0; s < C::CS; ++s) {
      float v[4];
      bf16x4_to_f32(d.cb[s], v);
#pragma unroll
      for (int e = 0; e < 4; ++e) pc = fmaf(v[e], k.Cc[s][e], pc);
    }
    if constexpr (C::CH) {
      float v[2];
      bf16x2_to_f32(d.cbh, v);
      pc = fmaf(v[0], k.Cch[0], pc);
      pc = fmaf(v[1], k.Cch[1], pc);
    }
  } else if constexpr (C::SEG8) {
#pragma unroll
    for (int s = 0; s < C::CS; ++s) {
      float v[4];
      fp8x4_to_f32(d.c8[s], v);
#pragma unroll
      for (int e = 0; e < 4; ++e) pc = fmaf(v[e], k.Cc[s][e], pc);
    }
    const f2 h = __builtin_amdgcn_cvt_pk_f32_fp8((int)d.c8h, false);
    pc = fmaf(h.x, k.Cch[0], pc);
    pc = fmaf(h.y, k.Cch[1], pc);
    pc *= d.sc;
  } else if constexpr (C::E4M3) {
#pragma unroll
    for (int i = 0; i < C::WORDS; ++i) {
      float v[4];
      fp8x4_to_f32(d.cw[i], v);
#pragma unroll
      for (int e = 0; e < 4; ++e) pc = fmaf(v[e], k.Cq[4 * i + e], pc);
    }
    pc *= d.sc;
  }
  return pc;
}

// Hot columns of one unit: decay-and-update in registers, store, and the lane's
// readout partial.
template <int K, int COLD>
__device__ __forceinline__ float hot_update(const StepArgs& a, size_t row, int q, UnitRaw<K, COLD>& d,
                                            const float* __restrict__ hd, const Coef<K, COLD>& k) {
  using C = Cfg<K, COLD>;
  const float uu = hd[HD_DT] * d.xp;
  const float dec = hd[HD_DECAY];
  float ph = 0.f;
  f4* hp = reinterpret_cast<f4*>(a.hot + row * K) + q;
#pragma unroll
  for (int s = 0; s < C::HS; ++s) {
    f4 v = d.hv[s];
    v.x = fmaf(v.x, dec, uu * k.Bh[s][0]);
    v.y = fmaf(v.y, dec, uu * k.Bh[s][1]);
    v.z = fmaf(v.z, dec, uu * k.Bh[s][2]);
    v.w = fmaf(v.w, dec, uu * k.Bh[s][3]);
    ph = fmaf(v.x, k.Ch[s][0], ph);
    ph = fmaf(v.y, k.Ch[s][1], ph);
    ph = fmaf(v.z, k.Ch[s][2], ph);
    ph = fmaf(v.w, k.Ch[s][3], ph);
    st_stream(v, hp + 8 * s);
  }
  if constexpr (C::HH) {
    f2 v = d.hh;
    v.x = fmaf(v.x, dec, uu * k.Bhh[0]);
    v.y = fmaf(v.y, dec, uu * k.Bhh[1]);
    ph = fmaf(v.x, k.Chh[0], ph);
    ph = fmaf(v.y, k.Chh[1], ph);
    st_stream(v, reinterpret_cast<f2*>(a.hot + row * K + 32 * C::HS) + q);
  }
  return ph;
}

// The exact readout's correction for row p of head (slot sh, request rh):
// sum_j cw_j x_j[p] over the window j = 0 .. m-1, the buffered tokens at ring positions
// pos - (m-1) + j and, last, this token (x = xcur); cw_j = w_j s_j with the window weight
// w_j = exp(sum_{l>j} a_l) dt_j (a_l = dt_l A) and s_j = C'_cold . B'_j from the prep kernel,
// scale/v4_native_decode.py:89-104. The window is at most 64 tokens, one per lane: lane j
// loads the 16 bytes of buffered x token j holds for the wave's 8 rows (p & ~7 ..), its dt
// (the ring's, this token's from the head scalars) and s_j; a suffix sum over the lanes
// gives the weights, and three exchange steps over lane bits 5, 4, 3 leave each lane its
// own row's share of 8 of the 64 products (lane l's row is l >> 3); the row's 8 lanes are
// summed with the rest of the readout, lane q = 0 adding this token's term. (Eight 2-byte
// loads per lane, token q + 8u for row p, ran the 9B-shape readout at c = 64 10.6 ms
// against 7.9 for the stale one.) The loads and the sum are separate so a kernel with
// registers to spare issues the loads with its state loads.
struct CorrRaw {
  uint4 xv;  // buffered x of window token `lane` for the wave's 8 rows (zero past m - 2)
  float dt;  // dt of window token `lane` (zero past m - 1)
  float s;   // s of window token `lane` (zero past m - 1)
};
__device__ __forceinline__ void corr_load(const StepArgs& a, const float* __restrict__ hd, size_t sh, size_t rh,
                                          int p, int q, CorrRaw& cr) {
  const int m = (int)hd[HD_M], c = a.c, lane = ((p & 7) << 3) | q;
  const int H = a.H, h = (int)(rh % H);
  // window token j sits at ring position pos - (m - 1) + j
  const int j0 = (int)hd[HD_POS] - (m - 1);
  const uint16_t* rx = a.ring_x + xring(a, sh, j0 + lane, p & ~7);
  const float* sw = Ws(a.ws, a.b, H, a.G, c).s + ((rh / H) * a.G + h / a.HG) * c;
  cr.s = lane < m ? sw[lane] : 0.f;
  cr.dt = lane < m - 1 ? a.ring_dt[sh * c + (j0 + lane)] : lane == m - 1 ? hd[HD_DT] : 0.f;
  cr.xv = lane < m - 1 ? *reinterpret_cast<const uint4*>(rx) : make_uint4(0u, 0u, 0u, 0u);
}
__device__ __forceinline__ float corr_sum(const float* __restrict__ hd, int p, int q, const CorrRaw& cr, float xcur) {
  const int m = (int)hd[HD_M], lane = ((p & 7) << 3) | q;
  // w_j = exp(sum_{l>j} a_l) dt_j: an inclusive suffix sum of a_l over the lanes (zero past
  // m - 1), shifted down by one lane
  float su = cr.dt * hd[HD_AH];
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float t = __shfl_down(su, d);
    if (lane + d < 64) su += t;
  }
  su = __shfl_down(su, 1);
  const float cw = expf(lane < 63 ? su : 0.f) * cr.dt * cr.s;
  const uint32_t xw[4] = {cr.xv.x, cr.xv.y, cr.xv.z, cr.xv.w};
  float v[8];  // w_j x_j[r] for the wave's rows r = 0 .. 7
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = cw * __uint_as_float(xw[i] << 16);
    v[2 * i + 1] = cw * __uint_as_float(xw[i] & 0xffff0000u);
  }
  // keep the half of the rows whose bit matches the lane's, add the partner's share of it
  const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
  float s4[4], s2[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) s4[i] = (b5 ? v[4 + i] : v[i]) + __shfl_xor(b5 ? v[i] : v[4 + i], 32);
#pragma unroll
  for (int i = 0; i < 2; ++i) s2[i] = (b4 ? s4[2 + i] : s4[i]) + __shfl_xor(b4 ? s4[i] : s4[2 + i], 16);
  float s = (b3 ? s2[1] : s2[0]) + dpp<0x128>(b3 ? s2[0] : s2[1]);  // row_ror:8, lane ^ 8
  // this token, window position m - 1 (cw of the lane that formed it)
  const float wl = m > 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cw), max(m, 1) - 1)) : 0.f;
  return q == 0 ? fmaf(wl, xcur, s) : s;
}
__device__ __forceinline__ float corr_partial(const StepArgs& a, const float* __restrict__ hd, size_t sh, size_t rh,
                                              int p, int q, float xcur) {
  CorrRaw cr;
  corr_load(a, hd, sh, rh, p, q, cr);
  return corr_sum(hd, p, q, cr, xcur);
}

// One unit of one token: hot columns, and (a head that does not flush at this token)
// the stale readout of its cold read copy and the ring append of x. A flushing head's
// cold columns are left to the flush kernel, which adds their readout to y.
// PRE: the exact readout's correction loads were issued with the state (cr), else here.
template <int K, int COLD, bool EXACT, bool PRE = false>
__device__ __forceinline__ void unit_compute(const StepArgs& a, size_t sh, size_t rh, int p, int q,
                                             UnitRaw<K, COLD>& d, uint16_t* rx, bool cold, const float* __restrict__ hd,
                                             const Coef<K, COLD>& k, const CorrRaw* cr = nullptr) {
  const size_t row = sh * a.P + p, yrow = rh * a.P + p;
  float part = hot_update<K, COLD>(a, row, q, d, hd, k);
  if constexpr (Cfg<K, COLD>::TIERED) {
    if (cold) part = fmaf(hd[HD_SNAPF], cold_partial<K, COLD>(d, k), part);
    if constexpr (EXACT) {
      if constexpr (PRE) part += corr_sum(hd, p, q, *cr, d.xp);
      else part += corr_partial(a, hd, sh, rh, p, q, d.xp);
    }
  }
  part = sum8(part);
  if (q == 0) {
    a.y[yrow] = fmaf(hd[HD_D], d.xp, part);
    if (rx) rx[p & 7] = d.xraw;  // ring append of x (tokens that do not flush; rx: the unit's granule)
  }
}

// Dot product of a lane's read-copy values with its C' (segment mapping).
template <int CS, bool CH>
__device__ __forceinline__ float seg_dot(const float (&r)[CS > 0 ? CS : 1][4], const float (&rh)[2],
                                         const float (*cc)[4], const float* cch) {
  float pc = 0.f;
#pragma unroll
  for (int s = 0; s < CS; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) pc = fmaf(r[s][e], cc[s][e], pc);
  if constexpr (CH) {
    pc = fmaf(rh[0], cch[0], pc);
    pc = fmaf(rh[1], cch[1], pc);
  }
  return pc;
}

// Write the new cold values of one row in the segment mapping (v: full segments, vh: the
// half segment of k_hot = 16): the fp32 copy, the single bf16 copy (RNE), or the master
// (fp32, or bf16 by RNE) and the bf16 / e4m3 read copy quantized from the master's values.
// RD: returns the lane's readout partial of the read copy as stored (C' in the segment
// mapping: cc [CS][4], cch [2]; e4m3 times the row scale), else 0.
template <int COLD, int CS, bool CH, bool RD = false>
__device__ __forceinline__ float cold_store(const StepArgs& a, size_t row, int q, const float (&v)[CS > 0 ? CS : 1][4],
                                            const float (&vh)[2], const float (*cc)[4] = nullptr,
                                            const float* cch = nullptr) {
  constexpr int NC = CS * 32 + (CH ? 16 : 0);
  float pc = 0.f;
  if constexpr (COLD == NSSM_COLD_FP32) {
    float* rp = static_cast<float*>(a.cold) + row * NC;
    f4* p = reinterpret_cast<f4*>(rp) + q;
#pragma unroll
    for (int s = 0; s < CS; ++s) st_stream(f4{v[s][0], v[s][1], v[s][2], v[s][3]}, p + 8 * s);
    if constexpr (CH) st_stream(f2{vh[0], vh[1]}, reinterpret_cast<f2*>(rp + 32 * CS) + q);
    if constexpr (RD) pc = seg_dot<CS, CH>(v, vh, cc, cch);
  } else if constexpr (COLD == NSSM_COLD_BF16_SINGLE) {
    uint16_t* base = static_cast<uint16_t*>(a.cold);
    u2v* p = reinterpret_cast<u2v*>(base + blk16(row, 4 * q, NC));
    float r[CS > 0 ? CS : 1][4], rh[2] = {0.f, 0.f};
#pragma unroll
    for (int s = 0; s < CS; ++s) {
      const u2v t = f32x4_to_bf16(v[s][0], v[s][1], v[s][2], v[s][3]);
      st_stream(t, p + kBlkSeg * s);
      bf16x4_to_f32(t, r[s]);
    }
    if constexpr (CH) {
      const uint32_t t = f32x2_to_bf16(vh[0], vh[1]);
      st_stream(t, reinterpret_cast<uint32_t*>(base + blk16(row, 32 * CS + 2 * q, NC)));
      bf16x2_to_f32(t, rh);
    }
    if constexpr (RD) pc = seg_dot<CS, CH>(r, rh, cc, cch);
  } else {
    float w[CS > 0 ? CS : 1][4], wh[2];  // the master's values
    if constexpr (COLD == NSSM_COLD_FP8_BF16M) {
      uint16_t* base = static_cast<uint16_t*>(a.master);
      u2v* pm = reinterpret_cast<u2v*>(base + blk16(row, 4 * q, NC));
#pragma unroll
      for (int s = 0; s < CS; ++s) {
        const u2v t = f32x4_to_bf16(v[s][0], v[s][1], v[s][2], v[s][3]);
        st_stream(t, pm + kBlkSeg * s);
        bf16x4_to_f32(t, w[s]);
      }
      if constexpr (CH) {
        const uint32_t t = f32x2_to_bf16(vh[0], vh[1]);
        st_stream(t, reinterpret_cast<uint32_t*>(base + blk16(row, 32 * CS + 2 * q, NC)));
        bf16x2_to_f32(t, wh);
      }
    } else {
      float* rp = static_cast<float*>(a.master) + row * NC;
      f4* pm = reinterpret_cast<f4*>(rp) + q;
#pragma unroll
      for (int s = 0; s < CS; ++s) {
        st_stream(f4{v[s][0], v[s][1], v[s][2], v[s][3]}, pm + 8 * s);
#pragma unroll
        for (int e = 0; e < 4; ++e) w[s][e] = v[s][e];
      }
      if constexpr (CH) {
        st_stream(f2{vh[0], vh[1]}, reinterpret_cast<f2*>(rp + 32 * CS) + q);
        wh[0] = vh[0];
        wh[1] = vh[1];
      }
    }
    if constexpr (COLD == NSSM_COLD_BF16) {
      uint16_t* base = static_cast<uint16_t*>(a.cold);
      u2v* p = reinterpret_cast<u2v*>(base + blk16(row, 4 * q, NC));
      float r[CS > 0 ? CS : 1][4], rh[2] = {0.f, 0.f};
#pragma unroll
      for (int s = 0; s < CS; ++s) {
        const u2v t = f32x4_to_bf16(w[s][0], w[s][1], w[s][2], w[s][3]);
        st_stream(t, p + kBlkSeg * s);
        bf16x4_to_f32(t, r[s]);
      }
      if constexpr (CH) {
        const uint32_t t = f32x2_to_bf16(wh[0], wh[1]);
        st_stream(t, reinterpret_cast<uint32_t*>(base + blk16(row, 32 * CS + 2 * q, NC)));
        bf16x2_to_f32(t, rh);
      }
      if constexpr (RD) pc = seg_dot<CS, CH>(r, rh, cc, cch);
    } else {  // e4m3 with the per-row amax scale of scale/vllm_v4_patch.py:106-111
      float am = 0.f;
#pragma unroll
      for (int s = 0; s < CS; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) am = fmaxf(am, fabsf(w[s][e]));
      if constexpr (CH) am = fmaxf(am, fmaxf(fabsf(wh[0]), fabsf(wh[1])));
      am = max8(am);
      const float sc = am / 448.0f + 1e-12f;
      const QDiv qd(sc);
      uint8_t* rp = static_cast<uint8_t*>(a.cold) + row * NC;
      uint32_t* p = reinterpret_cast<uint32_t*>(rp) + q;
      float r[CS > 0 ? CS : 1][4], rh[2] = {0.f, 0.f};
#pragma unroll
      for (int s = 0; s < CS; ++s) {
        const uint32_t t = f32x4_to_fp8(qd(w[s][0]), qd(w[s][1]), qd(w[s][2]), qd(w[s][3]));
        st_stream(t, p + 8 * s);
        if constexpr (RD) fp8x4_to_f32(t, r[s]);
      }
      if constexpr (CH) {
        const int t = __builtin_amdgcn_cvt_pk_fp8_f32(qd(wh[0]), qd(wh[1]), 0, false);
        st_stream((uint16_t)t, reinterpret_cast<uint16_t*>(rp + 32 * CS) + q);
        if constexpr (RD) {
          const f2 h = __builtin_amdgcn_cvt_pk_f32_fp8(t, false);
          rh[0] = h.x;
          rh[1] = h.y;
        }
      }
      if (q == 0) a.scale[row] = sc;
      if constexpr (RD) pc = seg_dot<CS, CH>(r, rh, cc, cch) * sc;
    }
  }
  return pc;
}

// The read-copy values of master values v: bf16 RNE, or the e4m3 codes of v / sc decoded (qd
// divides by the row's stored scale sc; the caller multiplies the readout by sc). Between
// flushes the stored read copy is exactly this quantization of the unchanged master: the join
// and every flush write both from the same values, with the same conversions.
template <int COLD>
__device__ __forceinline__ void requant4(const float (&v)[4], const QDiv& qd, float (&r)[4]) {
  if constexpr (COLD == NSSM_COLD_BF16) bf16x4_to_f32(f32x4_to_bf16(v[0], v[1], v[2], v[3]), r);
  else fp8x4_to_f32(f32x4_to_fp8(qd(v[0]), qd(v[1]), qd(v[2]), qd(v[3])), r);
}
template <int COLD>
__device__ __forceinline__ void requant2(const float (&v)[2], const QDiv& qd, float (&r)[2]) {
  if constexpr (COLD == NSSM_COLD_BF16) {
    bf16x2_to_f32(f32x2_to_bf16(v[0], v[1]), r);
  } else {
    const f2 h = __builtin_amdgcn_cvt_pk_f32_fp8(__builtin_amdgcn_cvt_pk_fp8_f32(qd(v[0]), qd(v[1]), 0, false), false);
    r[0] = h.x;
    r[1] = h.y;
  }
}

// C' of the cold columns in the segment mapping (k.Cc, k.Cch), for a kernel whose unit reads
// its e4m3 copy in the contiguous mapping and needs the segment one only on a flush.
template <int K, int COLD>
__device__ __forceinline__ void coef_cold_seg(const float* wC, int q, Coef<K, COLD>& k) {
  using C = Cfg<K, COLD>;
#pragma unroll
  for (int s = 0; s < C::CS; ++s) {
    const f4 tc = *reinterpret_cast<const f4*>(wC + K + 32 * s + 4 * q);
    k.Cc[s][0] = tc.x; k.Cc[s][1] = tc.y; k.Cc[s][2] = tc.z; k.Cc[s][3] = tc.w;
  }
  if constexpr (C::CH) {
    const f2 tc = *reinterpret_cast<const f2*>(wC + K + 32 * C::CS + 2 * q);
    k.Cch[0] = tc.x; k.Cch[1] = tc.y;
  }
}

// One unit of a head that flushes at this token, in the stream kernel (short windows):
// hot columns, the stale readout, and the exact cold state at this token, the decayed
// snapshot plus the VALU replay of the staged window (sU [m][P] of this head,
// sBc [m][NC]), scale/v4_fused_decode.py:76-85. A single copy is read once (it is both the
// stale snapshot and the replay's start); beside a master (fused_requant) only the master is
// read, and the stale readout is formed from its values quantized again (requant4: the stored
// read copy, bit for bit), so the flush token moves no read-copy bytes in.
// TF (the teacher-forced readout): the cold term is the readout of the new state as stored
// (the read copy), times HD_SNAPF = 1, instead of the stale snapshot's.
// The master values of one unit row in the segment mapping (and, e4m3, the row scale), for
// a flushing head of a kind with a master: loaded with the hot columns, ahead of the window
// staging and its barrier.
template <int K, int COLD>
struct MasterRaw {
  using C = Cfg<K, COLD>;
  u2v m16[C::MASTER16 ? C::CSR : 1];
  uint32_t m16h;
  f4 m32[C::MASTER32 ? C::CSR : 1];
  f2 m32h;
  float sc;
};
template <int K, int COLD>
__device__ __forceinline__ void master_load(const StepArgs& a, size_t row, int q, MasterRaw<K, COLD>& mr) {
  using C = Cfg<K, COLD>;
  constexpr int NC = C::NC, CS = C::CS;
  if constexpr (C::MASTER16) {
    const u2v* pm = reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(a.master) + blk16(row, 4 * q, NC));
#pragma unroll
    for (int s = 0; s < CS; ++s) mr.m16[s] = ld_stream(pm + kBlkSeg * s);
    if constexpr (C::CH)
      mr.m16h = ld_stream(reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.master) +
                                                            blk16(row, 32 * CS + 2 * q, NC)));
  } else if constexpr (C::MASTER32) {
    const f4* pm = reinterpret_cast<const f4*>(static_cast<const float*>(a.master) + row * NC) + q;
#pragma unroll
    for (int s = 0; s < CS; ++s) mr.m32[s] = ld_stream(pm + 8 * s);
    if constexpr (C::CH)
      mr.m32h = ld_stream(reinterpret_cast<const f2*>(static_cast<const float*>(a.master) + row * NC + 32 * CS) + q);
  }
  if constexpr (C::E4M3) mr.sc = a.scale[row];
}

// Whether the fused replay of a kind with a master forms the stale readout from the master
// (requant4) instead of loading the read copy: where the stream kernel compiles without
// spills at its occupancy bound. The bf16 read copy at k_hot = 32 (64 registers) and the
// k_hot = 16 kinds (80) spill three registers around the replay loop that way, and keep
// the load.
template <int K, int COLD>
constexpr bool fused_requant() {
  return (Cfg<K, COLD>::MASTER32 || Cfg<K, COLD>::MASTER16) && K != 16 && !(K == 32 && COLD == NSSM_COLD_BF16);
}

template <int K, int COLD, bool EXACT, bool TF = false, bool LAG = false>
__device__ __forceinline__ void unit_compute_flush(const StepArgs& a, size_t sh, size_t rh, int p, int q,
                                                   UnitRaw<K, COLD>& d, const float* __restrict__ hd,
                                                   const Coef<K, COLD>& k, const float* sU, const float* sBc, int m,
                                                   int ldu, int pofs, const MasterRaw<K, COLD>* mr = nullptr) {
  using C = Cfg<K, COLD>;
  constexpr int NC = C::NC, CS = C::CS;
  constexpr bool kMaster = fused_requant<K, COLD>() && !LAG;  // the read copy was not loaded
  constexpr bool kRequant = kMaster && !TF;  // the stale readout from the master's values
  const size_t row = sh * a.P + p, yrow = rh * a.P + p;
  float part = hot_update<K, COLD>(a, row, q, d, hd, k);
  if constexpr (!TF && !kMaster) part = fmaf(hd[HD_SNAPF], cold_partial<K, COLD>(d, k), part);
  const float osc = kRequant && C::E4M3 ? (mr ? mr->sc : a.scale[row]) : 1.f;  // the stored row scale
  const QDiv oq(osc);
  float pc = 0.f;  // kRequant: the stale readout partial of the requantized master
  const float dtot = hd[HD_DTOT];
  float nvv[C::CSR][4], nvh[2] = {0.f, 0.f};
#pragma unroll
  for (int s = 0; s < CS; ++s) {
    float t[4];
    if constexpr (COLD == NSSM_COLD_FP32) {
      t[0] = d.cf[s].x; t[1] = d.cf[s].y; t[2] = d.cf[s].z; t[3] = d.cf[s].w;
    } else if constexpr (COLD == NSSM_COLD_BF16_SINGLE) {
      bf16x4_to_f32(d.cb[s], t);
    } else if constexpr (C::MASTER16) {
      bf16x4_to_f32(mr ? mr->m16[s] : ld_stream(reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(a.master) + blk16(row, 4 * q, NC)) + kBlkSeg * s), t);
    } else {  // fp32 master
      const f4 m4 = mr ? mr->m32[s] : ld_stream(reinterpret_cast<const f4*>(static_cast<const float*>(a.master) + row * NC) + q + 8 * s);
      t[0] = m4.x; t[1] = m4.y; t[2] = m4.z; t[3] = m4.w;
    }
    if constexpr (kRequant) {
      float r[4];
      requant4<COLD>(t, oq, r);
#pragma unroll
      for (int e = 0; e < 4; ++e) pc = fmaf(r[e], k.Cc[s][e], pc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) nvv[s][e] = t[e] * dtot;
  }
  if constexpr (C::CH) {
    float t[2];
    if constexpr (COLD == NSSM_COLD_FP32) {
      t[0] = d.cfh.x; t[1] = d.cfh.y;
    } else if constexpr (COLD == NSSM_COLD_BF16_SINGLE) {
      bf16x2_to_f32(d.cbh, t);
    } else if constexpr (C::MASTER16) {
      bf16x2_to_f32(mr ? mr->m16h : ld_stream(reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.master) +
                                                               blk16(row, 32 * CS + 2 * q, NC))), t);
    } else {
      const f2 m2 = mr ? mr->m32h : ld_stream(reinterpret_cast<const f2*>(static_cast<const float*>(a.master) + row * NC + 32 * CS) + q);
      t[0] = m2.x; t[1] = m2.y;
    }
    if constexpr (kRequant) {
      float r[2];
      requant2<COLD>(t, oq, r);
      pc = fmaf(r[0], k.Cch[0], pc);
      pc = fmaf(r[1], k.Cch[1], pc);
    }
    nvh[0] = t[0] * dtot;
    nvh[1] = t[1] * dtot;
  }
  if constexpr (kRequant) part = fmaf(hd[HD_SNAPF], C::E4M3 ? pc * osc : pc, part);
  for (int i = 0; i < m; ++i) {
    const float coef = sU[i * ldu + (p - pofs)];
    const float* bc = sBc + i * NC + 4 * q;
#pragma unroll
    for (int s = 0; s < CS; ++s) {
      const f4 bb = *reinterpret_cast<const f4*>(bc + 32 * s);
      nvv[s][0] = fmaf(coef, bb.x, nvv[s][0]);
      nvv[s][1] = fmaf(coef, bb.y, nvv[s][1]);
      nvv[s][2] = fmaf(coef, bb.z, nvv[s][2]);
      nvv[s][3] = fmaf(coef, bb.w, nvv[s][3]);
    }
    if constexpr (C::CH) {
      const f2 bb = *reinterpret_cast<const f2*>(sBc + i * NC + 32 * CS + 2 * q);
      nvh[0] = fmaf(coef, bb.x, nvh[0]);
      nvh[1] = fmaf(coef, bb.y, nvh[1]);
    }
  }
  if constexpr (TF)
    part = fmaf(hd[HD_SNAPF], cold_store<COLD, CS, C::CH, true>(a, row, q, nvv, nvh, k.Cc, k.Cch), part);
  else
    cold_store<COLD, CS, C::CH>(a, row, q, nvv, nvh);
  // the exact readout's correction, once the replay's registers are free (nothing else
  // adds to part in between, so the sum is the same)
  if constexpr (EXACT) part += corr_partial(a, hd, sh, rh, p, q, d.xp);
  part = sum8(part);
  if (q == 0) a.y[yrow] = fmaf(hd[HD_D], d.xp, part);
}

// Window of one head for the rows [p0, p0 + nr) of a unit workgroup, in LDS:
// sB[i][n] = B'_i[K + n] (the group's cold columns) and sU[i][r] = w_i x_i[p0 + r]; window
// token m - 1 is this token (B' from the workspace, x from the inputs), token i < m - 1 sits
// at ring position c - m + i (rb0 points at the B' ring row of window token 0, rx0 at the x
// ring element of window token 0, row 0; xs_tok, xs_unit: the x ring's strides).
template <int NC>
__device__ __forceinline__ void stage_unit_window(float* sB, float* sU, int m, int xs_tok, int xs_unit, int p0, int nr,
                                                  const float* rb0, const float* bcur, const uint16_t* rx0,
                                                  const uint16_t* xcur, const float* wgt, int tid, int nthr) {
  constexpr int NB4 = NC / 4;
  for (int i = tid; i < m * NB4; i += nthr) {
    const int e = i / NB4;
    const float* src = e < m - 1 ? rb0 + (size_t)e * NC : bcur;
    reinterpret_cast<f4*>(sB)[i] = *reinterpret_cast<const f4*>(src + 4 * (i - e * NB4));
  }
  for (int i = tid; i < m * nr; i += nthr) {
    const int e = i / nr, r = i - e * nr;
    const uint16_t xs = e < m - 1 ? rx0[(size_t)e * xs_tok + ((p0 + r) >> 3) * xs_unit + ((p0 + r) & 7)] : xcur[p0 + r];
    sU[i] = wgt[e] * bf2f(xs);
  }
}

// One unit of a head that does not flush and whose cold term the gated readout drops:
// hot columns, y = hot C'[:K] + D x, and the ring append of x; no cold column is read.
template <int K, int COLD>
__device__ __forceinline__ void unit_hot_only(const StepArgs& a, const float* __restrict__ hd, const Ws& ws, size_t sh,
                                           size_t rh, size_t pair, int p, int q) {
  UnitRaw<K, COLD> d;
  unit_load<K, COLD>(a, sh * a.P + p, rh * a.P + p, q, d, true);
  Coef<K, COLD> k;
  coef_load<K, COLD>(ws.B + pair * kN, ws.C + pair * kN, q, k);
  uint16_t* rx = a.ring_x + xring(a, sh, (int)hd[HD_POS], p & ~7);
  unit_compute<K, COLD, false>(a, sh, rh, p, q, d, rx, false, hd, k);
}

// Stream kernel: one unit (8 headdim rows of one head) per wave; a workgroup is UW waves
// on consecutive units of one head (UW divides P / 8), workgroups in request-major, head,
// row order, so the resident waves stream a compact window of the state. FUSED (short
// windows): a flushing head's cold columns are replayed here from an LDS copy of the
// window (the group's B' columns and w_i x_i of the workgroup's rows); otherwise the flush
// kernel does them and this kernel leaves them alone.
// Occupancy bound of the stream kernel (waves per SIMD it is compiled for). Without one
// the fused replay's registers leave 4 waves per SIMD for every launch; measured on MI355X
// (B = 256, 27 layers, ms per step): fp32 cold c = 4 at 8 waves 8.57 (at 6: 8.59); e4m3
// over a bf16 master (B = 448) spills at 8 (12.66) and runs 11.62 at 6; wider hot tiers
// spill above 6 (k_hot = 64) and 5 (k_hot = 96), and k_hot = 16 (14 cold columns per lane
// and the half segments' coefficients) above 6.
template <int K, int COLD>
constexpr int unit_waves_per_eu() {
  return K == 32 ? (Cfg<K, COLD>::E4M3 ? 6 : 8) : K == kN ? 8 : K == 16 || K == 64 ? 6 : K == 0 ? 6 : 5;
}

// GATED: the gated readout's variant, in which a head that prep marked HD_SKIP and that
// does not flush takes the hot-only path (the other variants never wait for that flag
// before their state loads).
// TF: the teacher-forced readout's variant (a flushing head reads the state it replays;
// the other heads read the snapshot as the stale variant does, with prep's factor).
// LAG: the lagged teacher-forced readout's (a stale readout with prep's factor): a head
// that does not flush reads the second read copy (the snapshot before the last); a flushing
// head reads the old read copy, stores it there and replaces the first.
template <int K, int COLD, bool FUSED, bool EXACT, bool GATED, bool TF = false, bool LAG = false>
__device__ __forceinline__ void unit_body(const StepArgs& a, const float* __restrict__ hd_ro) {
  using C = Cfg<K, COLD>;
  constexpr int NC = C::NC;
  constexpr bool TIERED = C::TIERED;
  const int tid = threadIdx.x, lane = tid & 63, q = lane & 7, rr = lane >> 3;
  const int uw = blockDim.x >> 6, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, P = a.P, c = a.c, nub = (P >> 3) / uw;
  constexpr bool kXcd = ((NSSM_XCD_KINDS >> COLD) & 1) || (!FUSED && ((NSSM_XCD_SPLIT_KINDS >> COLD) & 1));
  const int wg = kXcd ? xcd_order(blockIdx.x, a.HG * nub, a.b * a.G) : (int)blockIdx.x;
  const int ub = wg % nub, hb = wg / nub, h = hb % H, bi = hb / H, g = h / a.HG;
  const int p0 = ub * uw * 8, p = p0 + wave * 8 + rr;
  const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
  const size_t rh = (size_t)bi * H + h;
  if (slot < 0 || slot >= a.slots) {  // uniform over the workgroup
    if (q == 0) a.y[rh * P + p] = __builtin_nanf("");
    return;
  }
  const size_t sh = (size_t)slot * H + h, row = sh * P + p;
  const Ws ws(a.ws, a.b, H, a.G, c);
  // per-head scalars through the noalias argument (scalar loads), except for the stale
  // readout over fp32 cold (vector loads measured faster there). The exact readout's
  // buffered-x addresses depend on them, and a vector load in front of those costs every
  // wave a second dependent memory round trip.
  constexpr bool kVecHd = COLD == NSSM_COLD_FP32 && TIERED && !EXACT;
  const float* __restrict__ hd = (kVecHd ? static_cast<const float*>(ws.hd) : hd_ro) + rh * HD_STRIDE;
  const bool flushing = TIERED && hd[HD_FLUSH] != 0.f;  // uniform over the workgroup
  if constexpr (TIERED && GATED) {
    // a head whose cold term the gated readout drops reads no cold columns unless it
    // flushes (its own path, so the common one keeps its unconditional loads)
    if (!flushing && hd[HD_SKIP] != 0.f) {
      unit_hot_only<K, COLD>(a, hd, ws, sh, rh, (size_t)bi * a.G + g, p, q);
      return;
    }
  }
  // a flushing head's read copy is needed here only when the replay is fused and the copy is
  // the replay's start (a single copy); beside a master the fused replay reads the master alone
  constexpr bool kMaster = fused_requant<K, COLD>() && !LAG;
  constexpr bool kCorrPre = EXACT && !FUSED && TIERED;
  // Where the head scalars are scalar loads, each path issues its own loads after the flag,
  // so the common path's go out together (e4m3 over a bf16 master, B = 256: non-flush tokens
  // 162 -> 157 us, 5.87 -> 5.76 ms per 27-layer step; B = 448 10.17 -> 10.02). Over fp32
  // cold (a vector load of the flag) the hot columns' loads are issued ahead of the flag's
  // wait, shared by both paths (the split order: 8.45 -> 8.59 ms at the headline); so are
  // the gated and teacher-forced variants' (their replay spills in the split order).
  if constexpr (!kVecHd && !GATED && !TF) {
    if constexpr (FUSED && TIERED) {
      if (flushing) {
        UnitRaw<K, COLD> d;
        unit_load<K, COLD>(a, row, rh * P + p, q, d, kMaster);
        const float* wB = ws.B + ((size_t)bi * a.G + g) * kN;
        const float* wC = ws.C + ((size_t)bi * a.G + g) * kN;
        Coef<K, COLD> k;
        coef_load<K, COLD, C::SEGREAD || TF>(wB, wC, q, k);
        extern __shared__ float lds[];
        const int m = min(max((int)hd[HD_M], 1), c);
        const int nr = uw * 8;
        float* sBc = lds;           // [m][NC]
        float* sU = lds + c * NC;   // [m][nr]
        // beside a master, the master (and e4m3 row scale) loads go out with the hot columns'
        // ahead of the staging, so the window's and the state's latencies overlap (the e4m3
        // flush token over a bf16 master: 380 -> 365 us at B = 256, 662 -> 635 at B = 448)
        MasterRaw<K, COLD> mr;
        constexpr bool kEarly = kMaster;
        if constexpr (kEarly) master_load<K, COLD>(a, row, q, mr);
        stage_unit_window<NC>(sBc, sU, m, a.xs_tok, a.xs_unit, p0, nr,
                              a.ring_b + (((size_t)slot * a.G + g) * c + (c - m)) * NC, wB + K,
                              a.ring_x + xring(a, sh, c - m, 0), a.x + rh * P, ws.w + rh * c, tid, blockDim.x);
        // the stale readout of the requantized master takes C' in the segment mapping
        if constexpr (kMaster && !TF && C::CONTIG) coef_cold_seg<K, COLD>(wC, q, k);
        __syncthreads();
        if constexpr (LAG) lag_store<K, COLD>(a, row, q, d);
        unit_compute_flush<K, COLD, EXACT, TF, LAG>(a, sh, rh, p, q, d, hd, k, sU, sBc, m, nr, p0,
                                                    kEarly ? &mr : nullptr);
        return;
      }
    }
    UnitRaw<K, COLD> d;
    if constexpr (LAG) unit_load<K, COLD>(a, row, rh * P + p, q, d, flushing, a.cold2, a.scale2);
    else unit_load<K, COLD>(a, row, rh * P + p, q, d, flushing);
    CorrRaw cr;
    if constexpr (kCorrPre) corr_load(a, hd, sh, rh, p, q, cr);
    const float* wB = ws.B + ((size_t)bi * a.G + g) * kN;
    const float* wC = ws.C + ((size_t)bi * a.G + g) * kN;
    Coef<K, COLD> k;
    coef_load<K, COLD, C::SEGREAD>(wB, wC, q, k);
    uint16_t* rx = nullptr;
    if constexpr (TIERED) {
      if (!flushing) rx = a.ring_x + xring(a, sh, (int)hd[HD_POS], p & ~7);
    }
    if constexpr (kCorrPre)
      unit_compute<K, COLD, EXACT, true>(a, sh, rh, p, q, d, rx, !flushing, hd, k, &cr);
    else
      unit_compute<K, COLD, EXACT>(a, sh, rh, p, q, d, rx, !flushing, hd, k);
  } else {
    UnitRaw<K, COLD> d;
    if constexpr (LAG) {
      unit_load<K, COLD>(a, row, rh * P + p, q, d, flushing && !FUSED, flushing ? a.cold : a.cold2,
                         flushing ? a.scale : a.scale2);
    } else {
      unit_load<K, COLD>(a, row, rh * P + p, q, d, flushing && (!FUSED || kMaster));
    }
    // the exact readout's correction: without the fused replay there are registers to issue
    // its loads now, beside the state's, instead of a second round trip after them
    CorrRaw cr;
    if constexpr (kCorrPre) corr_load(a, hd, sh, rh, p, q, cr);
    const float* wB = ws.B + ((size_t)bi * a.G + g) * kN;
    const float* wC = ws.C + ((size_t)bi * a.G + g) * kN;
    Coef<K, COLD> k;
    coef_load<K, COLD, C::SEGREAD || (TF && FUSED)>(wB, wC, q, k);
    if constexpr (FUSED && TIERED) {
      if (flushing) {
        extern __shared__ float lds[];
        const int m = min(max((int)hd[HD_M], 1), c);
        const int nr = uw * 8;
        float* sBc = lds;           // [m][NC]
        float* sU = lds + c * NC;   // [m][nr]
        MasterRaw<K, COLD> mr;
        constexpr bool kEarly = kMaster;
        if constexpr (kEarly) master_load<K, COLD>(a, row, q, mr);
        stage_unit_window<NC>(sBc, sU, m, a.xs_tok, a.xs_unit, p0, nr,
                              a.ring_b + (((size_t)slot * a.G + g) * c + (c - m)) * NC, wB + K,
                              a.ring_x + xring(a, sh, c - m, 0), a.x + rh * P, ws.w + rh * c, tid, blockDim.x);
        if constexpr (kMaster && !TF && C::CONTIG) coef_cold_seg<K, COLD>(wC, q, k);
        __syncthreads();
        if constexpr (LAG) lag_store<K, COLD>(a, row, q, d);
        unit_compute_flush<K, COLD, EXACT, TF, LAG>(a, sh, rh, p, q, d, hd, k, sU, sBc, m, nr, p0,
                                                    kEarly ? &mr : nullptr);
        return;
      }
    }
    uint16_t* rx = nullptr;
    if constexpr (TIERED) {
      if (!flushing) rx = a.ring_x + xring(a, sh, (int)hd[HD_POS], p & ~7);
    }
    if constexpr (kCorrPre)
      unit_compute<K, COLD, EXACT, true>(a, sh, rh, p, q, d, rx, !flushing, hd, k, &cr);
    else
      unit_compute<K, COLD, EXACT>(a, sh, rh, p, q, d, rx, !flushing, hd, k);
  }
}

// (the exact readout's fused replay over a 32-column fp32 or bf16 hot tier keeps the
// correction's window weights beside the replay's registers: 8 waves spill there)
template <int K, int COLD, bool FUSED, bool EXACT>
constexpr int unit_any_waves_per_eu() {
  return EXACT && FUSED && K == 32 && unit_waves_per_eu<K, COLD>() == 8 ? 7 : unit_waves_per_eu<K, COLD>();
}
template <int K, int COLD, bool FUSED, bool EXACT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(unit_any_waves_per_eu<K, COLD, FUSED, EXACT>()))) unit_kernel(StepArgs a, const float* __restrict__ hd_ro) {
  unit_body<K, COLD, FUSED, EXACT, false>(a, hd_ro);
}
template <int K, int COLD, bool FUSED>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(unit_waves_per_eu<K, COLD>()))) unit_kernel_gated(StepArgs a, const float* __restrict__ hd_ro) {
  unit_body<K, COLD, FUSED, false, true>(a, hd_ro);
}
// (the teacher-forced flush readout keeps a second coefficient set: k_hot = 16 over e4m3
// spills above 5 waves)
template <int K, int COLD>
constexpr int unit_tf_waves_per_eu() {
  return K == 16 && Cfg<K, COLD>::E4M3 ? 5 : unit_waves_per_eu<K, COLD>();
}
template <int K, int COLD, bool FUSED>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(unit_tf_waves_per_eu<K, COLD>()))) unit_kernel_tf(StepArgs a, const float* __restrict__ hd_ro) {
  unit_body<K, COLD, FUSED, false, false, true>(a, hd_ro);
}
// (the lagged readout's fused replay also stores the old read copy: at k_hot = 32 over an
// fp32 hot tier, 8 waves spill)
template <int K, int COLD, bool FUSED>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(unit_any_waves_per_eu<K, COLD, FUSED, true>()))) unit_kernel_lag(StepArgs a, const float* __restrict__ hd_ro) {
  unit_body<K, COLD, FUSED, false, false, false, true>(a, hd_ro);
}

// Untiered step (the full fp32 state is the hot tier, K = N): one one-wave workgroup per 2
// headdim rows of one head, one float4 of state per lane (lane l: row p0 + (l >> 5),
// columns 4 (l & 31) .. +3); a row's C.h readout is a sum over its 32 lanes (three DPP steps
// within 8, a row mirror within 16, one swizzle across the two 16-lane halves). In-place RMW
// at this shape ran 6.73 TB/s in a skeleton over a 1.34 GB buffer, against 6.40 with four
// float4 per lane (the unit kernel's shape at K = N). Workgroups in request, head, row
// order. The arithmetic per element is the hot update's. Measured at the 9B shape, B = 256
// (414 us per launch): two or four row pairs per wave with the coefficients loaded once and
// the rows' y written by one store (WRITE_SIZE falls from 1.031 to 1.000 of the state and y
// bytes) 425 us; 4, 8, 16 or 40 consecutive workgroups on one XCD (whole y sectors per L2, so WRITE_SIZE
// at the algorithmic bytes) 435-447 us; without prep (each wave computing its head's dt
// and decay from the raw inputs, no rotation) 572 us.
__global__ void __launch_bounds__(64) fresh_kernel(StepArgs a, const float* __restrict__ hd_ro) {
  const int lane = threadIdx.x, cl = lane & 31;
  const int H = a.H, P = a.P, np = P >> 1;
  const int pp = blockIdx.x % np, hb = blockIdx.x / np, h = hb % H, bi = hb / H, g = h / a.HG;
  const int p = 2 * pp + (lane >> 5);
  const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
  const size_t rh = (size_t)bi * H + h;
  if (slot < 0 || slot >= a.slots) {  // uniform over the workgroup
    if (cl == 0) a.y[rh * P + p] = __builtin_nanf("");
    return;
  }
  f4* sp = reinterpret_cast<f4*>(a.hot + (((size_t)slot * H + h) * P + p) * kN) + cl;
  f4 v = ld_stream(sp);
  const float* __restrict__ hd = hd_ro + rh * HD_STRIDE;
  const Ws ws(a.ws, a.b, H, a.G, 0);
  const size_t pair = (size_t)bi * a.G + g;
  const f4 bv = *reinterpret_cast<const f4*>(ws.B + pair * kN + 4 * cl);
  const f4 cv = *reinterpret_cast<const f4*>(ws.C + pair * kN + 4 * cl);
  const float xp = bf2f(a.x[rh * P + p]);
  const float uu = hd[HD_DT] * xp, dec = hd[HD_DECAY];
  v.x = fmaf(v.x, dec, uu * bv.x);
  v.y = fmaf(v.y, dec, uu * bv.y);
  v.z = fmaf(v.z, dec, uu * bv.z);
  v.w = fmaf(v.w, dec, uu * bv.w);
  float part = v.x * cv.x;
  part = fmaf(v.y, cv.y, part);
  part = fmaf(v.z, cv.z, part);
  part = fmaf(v.w, cv.w, part);
  st_stream(v, sp);
  part = sum8(part);
  part += dpp<0x140>(part);       // row_mirror: lane i <-> 15 - i, the other 8 of the 16
  part += __shfl_xor(part, 16);   // the row's other 16 lanes
  if (cl == 0) a.y[rh * P + p] = fmaf(hd[HD_D], xp, part);
}

// ---------------------------------------------------------------------------
// flush: the cold tier of every (request, head) whose phase wraps at this token.
// Per item:
//   cold <- exp(sum a) cold + Delta,  Delta[p][n] = sum_i w_i x_i[p] B'_i[n]
// over the window (the buffered tokens and this one), scale/v4_fused_decode.py:76-85,
// and y += exp(glog) (stale read copy . C'[K:]) — the stream kernel wrote the hot part
// and D x of these heads' y and left their cold columns alone.
//
// Work split: prep flags each (request, group) pair with a flushing head. Every
// workgroup ranks the flagged pairs (a block-wide prefix count over the flags) and
// takes a contiguous range of the ranked items (pair rank r covers items r HG .. r HG +
// HG - 1, one per head), so F flushing heads spread over min(F, grid) workgroups whatever
// the requests' phases, and a workgroup flushes the heads of a pair one after another
// (their shared B' window and C' are staged once).
//
// Delta is contracted on the matrix cores as 16 x 16 tiles (p-tile pt, n-tile nt) of
// v_mfma_f32_16x16x32_bf16: A = (w B')^T (16 n x 32 tokens), B = x (32 tokens x 16 p). x
// is bf16 already; v = w B' (fp32) is split into three bf16 parts with hi + mid + lo == v
// exactly, so the three bf16 products per token are exact and accumulate in fp32: the
// accuracy of an fp32 contraction at a fraction of fp32 MFMA's issue time (per 64 tokens
// and tile, fp32 16x16x4: 16 steps of 32 cycles; bf16 16x16x32: 2 steps x 3 parts of 16).
// The window is staged in LDS by DMA fch tokens at a time (the whole window when it fits,
// all its loads in flight together; with two whole windows in LDS, the first item's window,
// state tiles and y in one round trip, and after each item's last barrier the window of the
// item after next and the next item's tiles and y, in flight during the next contraction).
// A wave owns one n-tile and up to kMfmaTiles consecutive
// p-tiles, so it builds the split A operand once per 32-token step for all of them (8
// tokens of one cold column per lane, read from the staged B' and weights); the x operand
// of each tile is two transposing LDS loads (ds_read_b64_tr_b16), and whole 32-token steps
// read both operands without per-token predicates (a chunk's last partial step reads the
// buffer's padding tokens and zeroes them). Lane (li, lk) of a tile holds
// Delta[pt*16 + li][nt*16 + 4 lk .. +3]; the state is read and written in that mapping: the
// pass's tiles are loaded before the contraction, every load is waited for once after it,
// and the new values of all tiles are formed before the first store, so the stores go out
// back to back and the pass's barrier publishes LDS only (the stores stay in flight). With
// two whole windows in LDS the flush kernel also forms each window's weights w_i =
// exp(sum_{l>i} a_l) dt_i and the total decay from the ring's dt (a 64-lane suffix scan,
// off the prep kernel's critical path). An e4m3 pass holds whole rows (the row scale
// needs all of a row's tiles). Per-tile readout partials and row maxima go through LDS and
// are summed in a fixed order.
// Measured on MI355X (9B shape, B = 256, c = 64, fp32 cold), a full flush (32768 heads):
// 965 us with the fp32 contraction, 810-850 with the three-part bf16 split, 714 with the
// shared A operand and conflict-free window, 689-697 with a pair's B' staged once,
// 661-681 with the transposing x loads, predicate-free steps and stores back to back,
// 576-592 with plain state accesses (ld_flush / st_flush: WRITE_SIZE per full flush 1.25 ->
// 1.00 GB; e4m3 over a bf16 master 931 -> 690 us, the bf16 read copy over an fp32 master
// 1046 -> 819); 555-590 with the pair flags carrying slot and window length, per-item
// offsets listed once, the next item's tiles loaded early and no scratch (the ragged
// batch's per-token launch, B = 384, ~768 heads: 27.5 -> 25.6 us). Shader-clock timestamps
// in an instrumented copy put the contraction at about 2,000 cycles of an item and most of
// the rest in the item's own instructions between its loads and the contraction, not in
// waits on memory. Tried and slower: one wave per tile row (P / 16
// waves per workgroup, 3 workgroups per CU, row scales and readouts reduced in the wave)
// 1004 us; the window staged transposed and pre-split in LDS by the workgroup (three bf16
// copies of w B', token-contiguous rows) 1239 us; six-wave workgroups (one per work unit)
// holding the next item's tiles in registers 809 us (only one such workgroup is resident per
// CU); the next item's tiles in registers with eight waves (spills) 801 us; two helper
// waves staging windows and writing y while six contract (ragged 33.8 us).
constexpr int kFlushWaves = 8;
constexpr int kFlushPerCU = 2;  // flush workgroups per CU (the kernel's occupancy: 4 waves per SIMD)
constexpr int kFlushList = 64;  // items a workgroup lists at a time

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));

// The three bf16 parts of each of 8 fp32 values: hi = bf16(v), mid = bf16(v - hi),
// lo = bf16(v - hi - mid), with hi + mid + lo == v exactly (each difference is exact in
// fp32, and what is left after two 8-bit parts fits the third) for |v| above 2^-100.
__device__ __forceinline__ void split3x8(const float (&v)[8], u4v& hi, u4v& mi, u4v& lo) {
  // the differences must round v itself, not be fused with the product that formed v
#pragma clang fp contract(off)
  uint32_t h[4], m[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float t[2];
    h[j] = f32x2_to_bf16(v[2 * j], v[2 * j + 1]);
    bf16x2_to_f32(h[j], t);
    const float r0 = v[2 * j] - t[0], r1 = v[2 * j + 1] - t[1];
    m[j] = f32x2_to_bf16(r0, r1);
    bf16x2_to_f32(m[j], t);
    l[j] = f32x2_to_bf16(r0 - t[0], r1 - t[1]);
  }
  hi = u4v{h[0], h[1], h[2], h[3]};
  mi = u4v{m[0], m[1], m[2], m[3]};
  lo = u4v{l[0], l[1], l[2], l[3]};
}

// The flush kernel's state accesses: a 16 x 16 tile row is 64 bytes of fp32, half of a
// 128-byte line whose other half another wave of the workgroup reads and writes at about the
// same time; plain accesses let L2 merge the halves (non-temporal ones went to HBM apart).
#ifndef NSSM_FLUSH_NT
#define NSSM_FLUSH_NT 0
#endif
template <class T>
__device__ __forceinline__ T ld_flush(const T* p) {
  if constexpr (NSSM_FLUSH_NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <class T>
__device__ __forceinline__ void st_flush(T v, T* p) {
  if constexpr (NSSM_FLUSH_NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Window layout. The contraction's lane group lk (16 lanes; lanes 0-31 and 32-63 are served
// by the 32 LDS banks in separate cycles) takes, in each 32-token step from ks, the tokens
// ks + 16 q + 4 lk + r (q = 0, 1; r = 0 .. 3) as operand element 4 q + r. B' rows of tokens
// 4 apart start on the same bank when a token's B' spans whole 32-bank rows (NC % 32 ==
// 0), so within a token with bit 2 set its 16-byte granules are XORed with 4 (16 floats:
// the other half of the banks; groups lk = 0 and 1 differ in that bit). x rows are read
// with gfx950's transposing LDS load, 4 consecutive tokens per 16-lane group: a row is
// flush_x_stride(P) bf16 long, P padded by 16 where P is a multiple of 32, so consecutive
// rows start 32 bytes apart modulo the 128 bytes of the banks.
template <int NC>
__host__ __device__ constexpr int flush_swz_b() { return NC % 32 == 0 ? 4 : 0; }
__host__ __device__ constexpr int flush_x_stride(int P) { return P + (P % 32 == 0 ? 16 : 0); }
// Floats of one window buffer of fa tokens: [fa][NC] B', [fa][SX] x (bf16), [fa] weights,
// C'[K:] of the readout, and two scalars of its item (A_h and the readout factor HD_SNAPF)
// padded to 4.
__host__ __device__ constexpr int flush_win_floats(int fa, int NC, int P) {
  return fa * NC + fa * flush_x_stride(P) / 2 + fa + NC + 4;
}

// Stage window tokens [k0, k0 + kn) of one head into LDS with gfx950's LDS DMA
// (global_load_lds: lane L of a wave instruction writes its granule at base + L * size,
// no registers in between): sB[e][n] = B'_tok[K + n] (16-byte granules), sX[e][p] =
// x_tok[p] as bf16, both in the bank layout above (tok = k0 + e),
// sW[e] = w_tok, and sC[n] = C'[K + n] of this token
// (the readout's coefficients, read after the contraction); given dtcur, sW[e] = dt_tok instead
// (the caller forms the weights); given sScal, sScal[0] = *scA, sScal[1] = *scE (the item's
// scalars). Window token m - 1 is this
// token (B' from the workspace, x from the inputs); token tok < m - 1 sits at ring
// position c - m + tok (rb0 points at the B' ring row of window token 0, rx0 at the x ring
// granule of window token 0, rows 0 .. 7; xs_tok, xs_unit: the x ring's strides). Wave w
// issues the instructions w, w + nw, ... of each block; the caller waits (vmcnt) and
// barriers. withB = false leaves B' and C' as they are (the buffer holds this pair's).
template <int NC>
__device__ __forceinline__ void stage_window_dma(float* sB, uint16_t* sX, float* sW, float* sC, int k0, int kn,
                                                 int m, int P, const float* rb0, const float* bcur,
                                                 const uint16_t* rx0, int xs_tok, int xs_unit,
                                                 const uint16_t* xcur, const float* wgt,
                                                 const float* cq, int wave, int lane, int nw, bool withB,
                                                 const float* dtcur = nullptr, float* sScal = nullptr,
                                                 const float* scA = nullptr, const float* scE = nullptr) {
  // (the lane index opaque: each lane condition below is formed here, not hoisted by the
  // caller's loops into a scalar lane mask held across them)
  asm volatile("" : "+v"(lane));
  constexpr int NB4 = NC / 4;  // 16-byte granules per token of B'
  const int nb = withB ? kn * NB4 : 0;
  for (int q = wave; q * 64 < nb; q += nw) {
    const int gi = q * 64 + lane;
    if (gi < nb) {
      const int e = gi / NB4, tok = k0 + e;
      const int gr = (gi - e * NB4) ^ (flush_swz_b<NC>() * ((e >> 2) & 1));  // the granule this slot holds
      const float* src = (tok < m - 1 ? rb0 + (size_t)tok * NC : bcur) + 4 * gr;
      __builtin_amdgcn_global_load_lds(NSSM_GLOBAL(src), NSSM_LOCAL(sB + q * 256), 16, 0, 0);
    }
  }
  // x: the buffered tokens of the chunk in 16-byte granules (8 bf16; ring rows are
  // 16-byte aligned; a row's padding granules are filled from its first, and never read),
  // this token (window token m - 1, from the inputs) in 4-byte ones
  const int SX = flush_x_stride(P), P8 = P >> 3, S8 = SX >> 3;
  const int nxr = max(0, min(kn, m - 1 - k0)) * S8;
  for (int q = wave; q * 64 < nxr; q += nw) {
    const int gi = q * 64 + lane;
    if (gi < nxr) {
      const int e = gi / S8, gr = gi - e * S8;
      __builtin_amdgcn_global_load_lds(
          NSSM_GLOBAL(rx0 + (size_t)(k0 + e) * xs_tok + (size_t)(gr < P8 ? gr : 0) * xs_unit), NSSM_LOCAL(sX + q * 512),
          16, 0, 0);
    }
  }
  const int wx = nw >= 3 ? nw - 3 : 0, wc = nw >= 2 ? nw - 2 : 0;  // the waves of this token's x and of C'
  if (wave == wx && m - 1 >= k0 && m - 1 < k0 + kn) {
    const int e = m - 1 - k0, P2 = P >> 1;
    for (int q = 0; q * 64 < P2; ++q) {
      const int gi = q * 64 + lane;
      if (gi < P2)
        __builtin_amdgcn_global_load_lds(NSSM_GLOBAL(xcur + 2 * gi), NSSM_LOCAL(sX + e * SX + q * 128), 4, 0, 0);
    }
  }
  if (wave == nw - 1 && lane < kn)  // weights, or (dtcur given; whole windows) the buffered dt and this one
    __builtin_amdgcn_global_load_lds(NSSM_GLOBAL(dtcur && lane == m - 1 ? dtcur : wgt + k0 + lane), NSSM_LOCAL(sW), 4,
                                     0, 0);
  if (withB && wave == wc && lane < NC / 4)
    __builtin_amdgcn_global_load_lds(NSSM_GLOBAL(cq + 4 * lane), NSSM_LOCAL(sC), 16, 0, 0);
  if (sScal && wave == nw - 1 && lane < 2)
    __builtin_amdgcn_global_load_lds(NSSM_GLOBAL(lane ? scE : scA), NSSM_LOCAL(sScal), 4, 0, 0);
}

// Workgroup barrier that publishes LDS only: the wave's global stores stay in flight
// (HIP's __syncthreads also waits for them). A wave that staged LDS by DMA waits for its
// own DMA (vmcnt) before it reaches this barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The LDS byte address of a pointer into LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Two transposing LDS loads (ds_read_b64_tr_b16, 16-bit elements) at byte offset OFF from a0
// and a1, and the wait for them, in one asm statement. Through the builtin the compiler waits
// for every outstanding global load before the first such load (it does not tell them from
// the LDS DMA of the other window buffer), so the state tiles and the next window could not
// be in flight during the contraction. The window read here was published by a barrier
// after its DMA had landed; the asm has side effects, so it stays after that barrier.
template <int OFF>
__device__ __forceinline__ void ds_read_tr16_pair_at(uint32_t a0, uint32_t a1, short4v& t0, short4v& t1) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %2 offset:%4\n\t"
      "ds_read_b64_tr_b16 %1, %3 offset:%4\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(t0), "=&v"(t1)
      : "v"(a0), "v"(a1), "i"(OFF));
}
// tile i of a row of 16-column tiles (32 bytes apart); i is a constant where it is unrolled
__device__ __forceinline__ void ds_read_tr16_pair(uint32_t a0, uint32_t a1, int i, short4v& t0, short4v& t1) {
  static_assert(kMfmaTiles <= 5, "one case per tile");
  switch (i) {
    case 0: ds_read_tr16_pair_at<0>(a0, a1, t0, t1); break;
    case 1: ds_read_tr16_pair_at<32>(a0, a1, t0, t1); break;
    case 2: ds_read_tr16_pair_at<64>(a0, a1, t0, t1); break;
    case 3: ds_read_tr16_pair_at<96>(a0, a1, t0, t1); break;
    default: ds_read_tr16_pair_at<128>(a0, a1, t0, t1); break;
  }
}

// The flush kernel's static LDS: a list's items, their scalars and element offsets (formed
// once per item by the thread that lists it, so the waves read them instead of each forming
// them with scalar divisions and 64-bit products), and the ranking's scratch.
struct FlushList {
  int item[kFlushList], slot[kFlushList], m[kFlushList];  // m = 0: nothing to flush
  int pair[kFlushList], head[kFlushList];                   // request * G + group, head
  float dtot[kFlushList], eg[kFlushList];                   // (chunked windows) total decay, readout factor
  long long orow[kFlushList];  // first state row: (slot H + head) P
  long long ord[kFlushList];   // ring dt of window token 0: (slot H + head) c + c - m
  long long orb[kFlushList];   // ring B' of window token 0: ((slot G + group) c + c - m) NC
  int pairOf[kFlushList + 1];  // the pairs of a list's ranks
  float dT[2];                 // total decay of each window buffer's item (fw)
  int wave[kFlushWaves];
};

__device__ __forceinline__ long long rfl64(long long v) {
  const int lo = __builtin_amdgcn_readfirstlane((int)(v & 0xffffffff));
  const int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
  return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// The flush kernel's work units of an item: (n-tile, block of ptw consecutive p-tiles), the
// blocks as many as fill the nw waves (at most kMfmaTiles p-tiles each); NT n-tiles, P / 16
// p-tiles.
__device__ __forceinline__ int flush_ptw(int P, int NT, int nw) {
  const int PT = P / 16;
  const int nblk0 = max((PT + kMfmaTiles - 1) / kMfmaTiles, min(PT, nw / NT));
  return (PT + nblk0 - 1) / nblk0;
}

// Tokens a window buffer holds for a chunk of fch tokens: the contraction reads whole
// 32-token steps (tokens past the chunk are read and dropped).
__host__ __device__ constexpr int flush_alloc_tokens(int fch) { return (fch + 31) & ~31; }

// TF (the teacher-forced readout): y gets the readout of the new state as stored (the new
// read copy; e4m3 partials formed after the row scale is known) instead of the old one's.
// LAG (the lagged teacher-forced readout): the stale readout of the old read copy, which is
// also stored to the tier's second read copy (cold2, scale2) before the first is replaced.
template <int K, int COLD, bool TF = false, bool LAG = false>
__global__ void __launch_bounds__(kFlushWaves * 64) __attribute__((amdgpu_waves_per_eu(kFlushPerCU * kFlushWaves / 4)))
flush_kernel(StepArgs a) {
  static_assert(!(TF && LAG), "the lagged readout reads the old snapshot");
  using C = Cfg<K, COLD>;
  constexpr int NC = C::NC, NT = C::NT, nw = kFlushWaves, nthr = nw * 64;
  // work units: (n-tile, block of ptw consecutive p-tiles), one per wave and pass; the
  // blocks are as many as fill the waves (at most kMfmaTiles p-tiles each), and an e4m3
  // pass holds whole blocks (its row scales need every n-tile of a row)
  constexpr int UPP = C::E4M3 ? (nw / NT) * NT : nw;  // units per pass
  static_assert(UPP >= NT, "a pass must hold a whole row");
  // the values the flush starts from: the single copy, or the master (fp32 or bf16)
  constexpr bool SRC16 = COLD == NSSM_COLD_BF16_SINGLE || C::MASTER16;
  extern __shared__ float lds[];
  // this workgroup's listed items and their scalars (loaded by the thread that lists
  // the item); sM = 0 marks an item with nothing to flush
  __shared__ FlushList sL;
  int(&sItem)[kFlushList] = sL.item;
  int(&sSlot)[kFlushList] = sL.slot;
  int(&sM)[kFlushList] = sL.m;
  float(&sDtot)[kFlushList] = sL.dtot;
  float(&sEg)[kFlushList] = sL.eg;
  int(&sPairOf)[kFlushList + 1] = sL.pairOf;
  float(&sDT)[2] = sL.dT;
  int(&sWave)[kFlushWaves] = sL.wave;
  int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int li = lane & 15, lk = lane >> 4;
  const int H = a.H, P = a.P, c = a.c, G = a.G, HG = a.HG, fch = a.fch;
  const int fa = flush_alloc_tokens(fch);
  const Ws ws(a.ws, a.b, H, G, c);
  // window buffer (flush_win_floats): two of them when the next item's window is staged during
  // this one's contraction (then every window is whole, m <= c <= fch)
  const bool pipe = a.fpipe != 0, fw = pipe && a.fw != 0;
  const int SX = flush_x_stride(P);
  const int wfl = flush_win_floats(fa, NC, P);
  auto scal = [&](int bf) { return lds + bf * wfl + fa * NC + fa * SX / 2 + fa + NC; };  // A_h, HD_SNAPF
  const int nbuf = pipe ? 2 : 1;
  float* sPart0 = lds + nbuf * wfl;        // [nbuf][P][NT] readout partials of the old read copy
  float* sAmx = sPart0 + nbuf * P * NT;    // [P][NT] row maxima of the new values (e4m3 only)
  const int PT = P / 16, ptw = flush_ptw(P, NT, nw), nunit = NT * ((PT + ptw - 1) / ptw);

  // 1. rank the flagged pairs: thread tid counts pairs [p0, p1) (whole int4 words of
  // the flag array, which is padded to a multiple of 4), keeping the flags of its first 64
  // pairs as a bit mask, then a block-wide exclusive prefix of the counts
  const int npair = a.b * G;
  const int per = (((npair + nthr - 1) / nthr) + 3) & ~3;
  const int p0 = min(tid * per, npair), p1 = min(p0 + per, npair);
  int cnt = 0;
  uint64_t fmask = 0;
  for (int p = p0; p < p1; p += 4) {
    const int4 f = *reinterpret_cast<const int4*>(ws.fg + p);
    const uint32_t bits = (uint32_t)(f.x != 0) | ((uint32_t)(p + 1 < p1 && f.y != 0) << 1) |
                          ((uint32_t)(p + 2 < p1 && f.z != 0) << 2) | ((uint32_t)(p + 3 < p1 && f.w != 0) << 3);
    if (p - p0 < 64) fmask |= (uint64_t)bits << (p - p0);
    cnt += __builtin_popcount(bits);
  }
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == 63) sWave[wave] = incl;
  __syncthreads();
  int rank0 = incl - cnt, total = 0;
#pragma unroll
  for (int w2 = 0; w2 < nw; ++w2) {
    const int s = sWave[w2];
    rank0 += w2 < wave ? s : 0;
    total += s;
  }
  const int fitems = total * HG;  // heads of flagged pairs (at most b H, far below 2^31: the workspace
                                  // holds HD_STRIDE floats per head)
  // each workgroup takes a contiguous range of the ranked items (consecutive heads of a
  // pair in a row: the pair's B' window is staged once for them)
  const int bx = blockIdx.x, grid = gridDim.x;
  const int per_wg = (fitems + grid - 1) / grid;
  const int ilo = min(bx * per_wg, fitems);
  const int nmine = min(ilo + per_wg, fitems) - ilo;
  int bkey0 = -1, bkey1 = -1;  // the pair whose B' and C' each window buffer holds (-1: none)

  // the state tiles of one pass of an item, in registers: issued early, used after the
  // contraction
  // (beside a master the old read copy is not loaded: it is the master's quantization, formed
  // again from the master tiles, requant4)
  f4 old[kMfmaTiles];
  u2v old16[SRC16 ? kMfmaTiles : 1];
  float rsc[C::E4M3 ? kMfmaTiles : 1];
  // this wave's work unit in the pass from unit u0: n-tile nt, p-tiles pt0 .. pt0 + npt - 1
  // (npt = 0: no unit in this pass)
  auto unit_of = [&](int u0, int& nt, int& pt0) {
    const int u = u0 + wave;
    nt = u % NT;
    pt0 = (u / NT) * ptw;
    return wave < UPP && u < nunit ? min(ptw, PT - pt0) : 0;  // wave-uniform
  };
  auto load_tiles = [&](int kk, int u0) {
    int nt, pt0;
    const int npt = unit_of(u0, nt, pt0);
    const size_t row0 = (size_t)rfl64(sL.orow[kk]);
    const void* src = C::SEG ? static_cast<const void*>(a.cold) : static_cast<const void*>(a.master);
#pragma unroll
    for (int i = 0; i < kMfmaTiles; ++i) {
      if (i < npt) {
        const size_t row = row0 + (pt0 + i) * 16 + li;
        const int col = nt * 16 + 4 * lk;
        if constexpr (SRC16)
          old16[i] = ld_flush(reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(src) + blk16(row, col, NC)));
        else
          old[i] = ld_flush(reinterpret_cast<const f4*>(static_cast<const float*>(src) + row * NC + col));
        if constexpr (C::E4M3) rsc[i] = a.scale[row];
      }
    }
  };

  // 2. the pairs of this workgroup's ranks R0 .. R1 (items ilo .. ilo + nmine - 1; item ci is
  // head ci % HG of the pair of rank ci / HG), recorded once in sPairOf by the threads that
  // own them, from their masks (a thread with more than 64 pairs reads the flags past them
  // again). When they are more than sPairOf holds (more than about kFlushList * HG items a
  // workgroup), each list below records its own ranks, reading the flags again.
  const int R0 = ilo / HG, R1 = nmine > 0 ? (ilo + nmine - 1) / HG : R0 - 1;
  const bool once = R1 - R0 < kFlushList + 1;
  auto record = [&](int r_lo, int r_hi, bool from_mask) {
    if (cnt > 0 && rank0 <= r_hi && rank0 + cnt > r_lo) {
      int r = rank0, p = p0;
      if (from_mask) {
        uint64_t mrem = fmask;
        while (mrem != 0 && r <= r_hi) {
          const int j = __builtin_ctzll(mrem);
          mrem &= mrem - 1;
          if (r >= r_lo) sPairOf[r - r_lo] = p0 + j;
          ++r;
        }
        p = p0 + 64;
      }
      for (; p < p1 && r <= r_hi; ++p) {
        if (ws.fg[p] == 0) continue;
        if (r >= r_lo) sPairOf[r - r_lo] = p;
        ++r;
      }
    }
  };
  if (once) record(R0, R1, true);

  for (int j0 = 0; j0 < nmine; j0 += kFlushList) {
    const int jn = min(kFlushList, nmine - j0);
    __syncthreads();  // the pairs are recorded; the previous list is consumed
    // list items ilo + j0 .. + jn - 1, one thread per item
    const int a0 = ilo + j0;
    const int r_lo = once ? R0 : a0 / HG;  // the rank sPairOf[0] holds
    if (!once) record(r_lo, (a0 + jn - 1) / HG, false);
    __syncthreads();
    if (tid < jn) {
      const int ci = a0 + tid;
      const int r = ci / HG, hh = ci - r * HG;
      const int p = sPairOf[r - r_lo];
      const int bi = p / G, g = p - bi * G;
      const int it = bi * H + g * HG + hh;
      // a positive flag carries the slot and the window length of every head of the pair
      // (prep's flush_flag): no head scalar is read here
      const int fl = ws.fg[p];
      const float* hd = ws.hd + (size_t)it * HD_STRIDE;
      int slot = fl >> 7, m = fl & 127;
      bool ok = slot < a.slots;
      if (fl <= 0) {
        slot = a.slot_ids ? a.slot_ids[bi] : bi;
        ok = slot >= 0 && slot < a.slots && hd[HD_FLUSH] != 0.f;
        m = (int)hd[HD_M];
      }
      const int mc = ok ? min(max(m, 1), c) : 0, h = g * HG + hh;
      sItem[tid] = it;
      sSlot[tid] = slot;
      sM[tid] = mc;
      sL.pair[tid] = p;
      sL.head[tid] = h;
      if (ok) {
        const long long sh = (long long)slot * H + h;
        sL.orow[tid] = sh * P;
        sL.ord[tid] = sh * c + (c - mc);
        sL.orb[tid] = (((long long)slot * G + g) * c + (c - mc)) * NC;
      }
      if (!pipe) {  // (whole windows stage these scalars with the window)
        sDtot[tid] = hd[HD_DTOT];
        sEg[tid] = hd[HD_SNAPF];
      }
    }
    __syncthreads();

    // 3. the listed items. Staging of item kk's whole window (tokens 0 .. m-1) into buffer
    // bf: window token m - 1 is this token (B' from the workspace, x from the inputs),
    // token i < m - 1 sits at ring position c - m + i.
    auto stage_item = [&](int kk, int bf) {
      const int m2 = __builtin_amdgcn_readfirstlane(sM[kk]), it2 = __builtin_amdgcn_readfirstlane(sItem[kk]);
      const int key = __builtin_amdgcn_readfirstlane(sL.pair[kk]), h2 = __builtin_amdgcn_readfirstlane(sL.head[kk]);
      const size_t od = (size_t)rfl64(sL.ord[kk]);
      const bool withB = (bf ? bkey1 : bkey0) != key;  // a pair's heads share its B' window and C'
      if (bf) bkey1 = key;
      else bkey0 = key;
      float* wb = lds + bf * wfl;
      stage_window_dma<NC>(wb, reinterpret_cast<uint16_t*>(wb + fa * NC), wb + fa * NC + fa * SX / 2,
                           wb + fa * NC + fa * SX / 2 + fa, 0, m2, m2, P, a.ring_b + (size_t)rfl64(sL.orb[kk]),
                           ws.B + (size_t)key * kN + K,
                           a.ring_x + (size_t)rfl64(sL.orow[kk]) * c + (size_t)(c - m2) * a.xs_tok, a.xs_tok, a.xs_unit,
                           a.x + (size_t)it2 * P,
                           fw ? a.ring_dt + od : ws.w + (size_t)it2 * c, ws.C + (size_t)key * kN + K, wave, lane,
                           nw, withB,
                           fw ? ws.hd + (size_t)it2 * HD_STRIDE + HD_DT : nullptr, scal(bf), a.A + h2,
                           ws.hd + (size_t)it2 * HD_STRIDE + HD_SNAPF);
    };
    // fw: the window weights of item kk in buffer bf from its staged dt (one wave, after
    // its own DMA of them has landed): a_i = dt_i A_h, w_i = exp(sum_{l>i} a_l) dt_i (a
    // suffix scan over the window's lanes, at most 64 tokens) and the total decay
    // exp(sum_l a_l), as the reference's flush (scale/v4_fused_decode.py:76-79)
    auto form_weights = [&](int kk, int bf) {
      float* sWb = lds + bf * wfl + fa * NC + fa * SX / 2;
      const int mm = sM[kk];
      int ln = lane;
      asm volatile("" : "+v"(ln));  // (lane conditions formed here, not hoisted as lane masks)
      const float d = ln < mm ? sWb[ln] : 0.f;
      float incl = d * scal(bf)[0];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float v = __shfl_down(incl, o);
        if (ln + o < 64) incl += v;
      }
      const float after = __shfl_down(incl, 1);  // sum over l > lane
      if (ln < mm) sWb[ln] = expf(ln + 1 < mm ? after : 0.f) * d;
      if (ln == 0) sDT[bf] = expf(incl);
    };
    auto next_item = [&](int kk) {  // the first listed item from kk on with a window
      while (kk < jn && sM[kk] == 0) ++kk;
      return kk;
    };
    int buf = 0;
    float yv = 0.f;  // the item's y (hot part and D x, from the stream kernel)
    if (pipe) {
      // the first item's window, state tiles (its first pass) and y, in one round trip;
      // then the second item's window, in flight during the first item's contraction
      const int k1 = next_item(0);
      if (k1 < jn) {
        stage_item(k1, 0);
        load_tiles(k1, 0);
        if (tid < P) yv = a.y[(size_t)sItem[k1] * P + tid];
        __builtin_amdgcn_s_waitcnt(0);
        if (fw && wave == nw - 1) form_weights(k1, 0);
        __syncthreads();
        const int k2 = next_item(k1 + 1);
        if (k2 < jn) stage_item(k2, 1);
      }
    }
    for (int k = next_item(0); k < jn; k = next_item(k + 1)) {
      // the lane indices, opaque to the compiler from here on: per-lane conditions are formed
      // where they are used instead of hoisted out of the item loop as 64-bit lane masks held
      // in scalar registers for the whole loop (which spilled them)
      asm volatile("" : "+v"(tid), "+v"(lane), "+v"(li), "+v"(lk));
      const int m = __builtin_amdgcn_readfirstlane(sM[k]);  // > 0; these are workgroup-uniform
      const int it = __builtin_amdgcn_readfirstlane(sItem[k]), pr = __builtin_amdgcn_readfirstlane(sL.pair[k]);
      const float dtot = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fw ? sDT[buf] : sDtot[k])));
      const float eg = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(pipe ? scal(buf)[1] : sEg[k])));
      const size_t row0 = (size_t)rfl64(sL.orow[k]);
      if (!pipe && tid < P) yv = a.y[(size_t)it * P + tid];
      float* sBc = lds + buf * wfl;
      uint16_t* sX = reinterpret_cast<uint16_t*>(sBc + fa * NC);
      float* sW = sBc + fa * NC + fa * SX / 2;
      const float* sCq = sW + fa;  // C'[K:]
      float* sPart = sPart0 + buf * P * NT;
      const bool whole = m <= fch;  // the window fits in LDS: staged once

      // the passes (at least one: P >= 16; one at the 9B shape), as a do-while so the compiler
      // sees that the pass's wait below separates every prefetch of the state tiles from the next
      int u0 = 0;
      do {
        int nt, pt0;
        const int npt = unit_of(u0, nt, pt0);
        asm volatile("" : "+v"(tid), "+v"(lane), "+v"(li), "+v"(lk));  // (as at the item's top)
        if (!pipe || u0 > 0) load_tiles(k, u0);  // (whole windows: the first pass's were loaded before)
        f4 acc[kMfmaTiles];
#pragma unroll
        for (int i = 0; i < kMfmaTiles; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};
        // One 32-token k-step of A = (w B')^T (16 n x 32 tokens) against B = x (32 tokens x
        // 16 p), tokens ks .. ks + 31 of the staged chunk of kn tokens: lane (li, lk) builds
        // row / column li, tokens ks + lk + 4 j (j = 0 .. 7) of each operand (any assignment
        // of tokens to k that A and B share gives the same product), A as the three bf16
        // parts of v = w B' (hi + mid + lo == v), so the three bf16 products per token are
        // exact and sum in fp32. A is built once per step for all of the wave's tiles (they
        // share the n-tile). A step inside the chunk reads its operands unconditionally;
        // the last step of a chunk that is not a whole number of steps (tail) reads the
        // buffer's tokens past the chunk (held in the allocation, flush_alloc_tokens) and
        // zeroes them in both operands.
        auto kstep = [&](int ks, int kn, auto tail_tag, auto ntiles) {
          constexpr bool TAIL = decltype(tail_tag)::value;
          const int kg = ks + 4 * lk;  // this lane group's tokens: kg + 16 q + r
          // A: this lane's row li of w B' over its 8 tokens, through the bank swizzle (bit 2
          // of kg + 16 q + r is lk & 1); the empty asm keeps the compiler from turning the
          // per-token addresses into loop-carried registers (token (q, r) is then an
          // immediate offset, (16 q + r) NC floats)
          int bo = kg * NC + 4 * ((4 * nt + (li >> 2)) ^ (flush_swz_b<NC>() * (lk & 1))) + (li & 3);
          asm volatile("" : "+v"(bo));
          const f4 w0 = *reinterpret_cast<const f4*>(sW + kg), w1 = *reinterpret_cast<const f4*>(sW + kg + 16);
          float v[8];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int e = 4 * q + r;
              v[e] = (q ? w1[r] : w0[r]) * sBc[bo + (16 * q + r) * NC];
              if constexpr (TAIL) v[e] = kg + 16 * q + r < kn ? v[e] : 0.f;
            }
          }
          u4v hv, mv, lv;
          split3x8(v, hv, mv, lv);
          __builtin_amdgcn_sched_barrier(0);
          // B = x of each tile by two transposing loads (ds_read_b64_tr_b16: within a 16-lane
          // group, lane j's element r comes from lane (j >> 2) + 4 r, element j & 3): group
          // lane li reads headdim rows 16 (pt0 + i) + 4 (li & 3) .. + 3 of token kg + 16 q +
          // (li >> 2), so lane li gets row 16 (pt0 + i) + li of tokens kg + 16 q + r as
          // elements 4 q + r, the tokens of A's elements. All loads first, then the products
          // part by part across the tiles (independent accumulators back to back).
          int xo = (kg + (li >> 2)) * SX + 16 * pt0 + 4 * (li & 3);
          asm volatile("" : "+v"(xo));
          const uint32_t xa0 = lds_addr(sX + xo), xa1 = lds_addr(sX + xo + 16 * SX);
#pragma unroll
          for (int i = 0; i < kMfmaTiles; ++i) {
            if (i < ntiles) {  // wave-uniform
              u2v h2[2];
              short4v tq[2];
              ds_read_tr16_pair(xa0, xa1, i, tq[0], tq[1]);
#pragma unroll
              for (int q = 0; q < 2; ++q) {
                short4v t = tq[q];
                if constexpr (TAIL) {
#pragma unroll
                  for (int r = 0; r < 4; ++r) t[r] = kg + 16 * q + r < kn ? t[r] : (short)0;
                }
                h2[q] = __builtin_bit_cast(u2v, t);
              }
              const bf16x8 xb = __builtin_bit_cast(bf16x8, (u4v{h2[0].x, h2[0].y, h2[1].x, h2[1].y}));
              acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, hv), xb, acc[i], 0, 0, 0);
              acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, mv), xb, acc[i], 0, 0, 0);
              acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, lv), xb, acc[i], 0, 0, 0);
            }
          }
        };
        for (int k0 = 0; k0 < m; k0 += fch) {
          const int kn = min(fch, m - k0);
          if (!pipe && (!whole || u0 == 0)) {  // a whole window is staged once, in the first pass
            __syncthreads();  // the previous chunk (or item: window and partials) is consumed
            // whole windows keep the pair's B' and C' from its previous head
            const bool withB = !whole || bkey0 != pr;
            bkey0 = whole ? pr : -1;
            stage_window_dma<NC>(sBc, sX, sW, sW + fa, k0, kn, m, P, a.ring_b + (size_t)rfl64(sL.orb[k]),
                                 ws.B + (size_t)pr * kN + K,
                                 a.ring_x + (size_t)rfl64(sL.orow[k]) * c + (size_t)(c - m) * a.xs_tok, a.xs_tok,
                                 a.xs_unit, a.x + (size_t)it * P,
                                 ws.w + (size_t)it * c, ws.C + (size_t)pr * kN + K, wave, lane, nw,
                                 withB);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA has landed in LDS
            __syncthreads();
          }
          if (npt > 0) {
            int ks = 0;
            for (; ks + 32 <= kn; ks += 32) kstep(ks, kn, std::false_type{}, npt);
            if (ks < kn) kstep(ks, kn, std::true_type{}, npt);
          }
        }
        // Every load of this wave is waited for here, before its first store: the pass's
        // state tiles, with pipe this wave's part of the next window, and the previous
        // item's stores (loads and stores share one counter). The stores below then go out
        // back to back, and the barrier after them waits for LDS only.
        __builtin_amdgcn_s_waitcnt(0);
        if (fw && u0 == 0 && wave == nw - 1) {  // the next item's weights (its dt staged above; published below)
          const int knext = next_item(k + 1);
          if (knext < jn) form_weights(knext, buf ^ 1);
        }
        // new = total decay x old + Delta (into acc; the bf16 copies rounded), and the
        // readout partial of the old read copy
#pragma unroll
        for (int i = 0; i < kMfmaTiles; ++i) {
          if (i < npt) {
            const int p = (pt0 + i) * 16 + li, col = nt * 16 + 4 * lk;
            const f4 cq = *reinterpret_cast<const f4*>(sCq + col);
            if constexpr (SRC16) {
              float o4[4];
              bf16x4_to_f32(old16[i], o4);
              old[i] = f4{o4[0], o4[1], o4[2], o4[3]};
            }
            float rd[4];
            float rscale = 1.f;
            if constexpr (C::SEG) {  // the single copy is the read copy
              rd[0] = old[i].x; rd[1] = old[i].y; rd[2] = old[i].z; rd[3] = old[i].w;
            } else {  // the master's read copy: bf16 RNE, or e4m3 at the stored row scale
              const float ov[4] = {old[i].x, old[i].y, old[i].z, old[i].w};
              if constexpr (C::E4M3) rscale = rsc[i];
              requant4<COLD>(ov, QDiv(rscale), rd);
            }
            if constexpr (LAG) {  // the old read copy becomes the lagged one
              const size_t row = row0 + p;
              if constexpr (COLD == NSSM_COLD_FP32) {
                st_flush(old[i], reinterpret_cast<f4*>(static_cast<float*>(a.cold2) + row * NC + col));
              } else if constexpr (C::B16) {  // (rd holds bf16 values: this conversion is exact)
                st_flush(f32x4_to_bf16(rd[0], rd[1], rd[2], rd[3]),
                         reinterpret_cast<u2v*>(static_cast<uint16_t*>(a.cold2) + blk16(row, col, NC)));
              } else {  // e4m3: the codes of the old values at the stored scale
                const QDiv qd(rscale);
                st_flush(f32x4_to_fp8(qd(old[i].x), qd(old[i].y), qd(old[i].z), qd(old[i].w)),
                         reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.cold2) + row * NC + col));
                if (nt == 0 && lk == 0) a.scale2[row] = rscale;
              }
            }
            float pc = rd[0] * cq.x;
            pc = fmaf(rd[1], cq.y, pc);
            pc = fmaf(rd[2], cq.z, pc);
            pc = fmaf(rd[3], cq.w, pc);
            f4 nv = acc[i];
            nv.x = fmaf(dtot, old[i].x, nv.x);
            nv.y = fmaf(dtot, old[i].y, nv.y);
            nv.z = fmaf(dtot, old[i].z, nv.z);
            nv.w = fmaf(dtot, old[i].w, nv.w);
            if constexpr (SRC16) {  // bf16 single copy or bf16 master: RNE (stored below as the
              // bf16 of these exact values), and the e4m3 copy is quantized from the rounded values
              float r4[4];
              bf16x4_to_f32(f32x4_to_bf16(nv.x, nv.y, nv.z, nv.w), r4);
              nv = f4{r4[0], r4[1], r4[2], r4[3]};
            }
            acc[i] = nv;
            if constexpr (COLD == NSSM_COLD_BF16) {
              if constexpr (TF) bf16x4_to_f32(f32x4_to_bf16(nv.x, nv.y, nv.z, nv.w), rd);  // the new read copy
            } else if constexpr (TF) {
              rd[0] = nv.x; rd[1] = nv.y; rd[2] = nv.z; rd[3] = nv.w;  // fp32 copy, or the rounded bf16 one
            }
            if constexpr (TF && !C::E4M3) {
              pc = rd[0] * cq.x;
              pc = fmaf(rd[1], cq.y, pc);
              pc = fmaf(rd[2], cq.z, pc);
              pc = fmaf(rd[3], cq.w, pc);
            }
            if constexpr (!(TF && C::E4M3)) {  // (teacher-forced e4m3: after the row scale below)
              pc += __shfl_xor(pc, 16);
              pc += __shfl_xor(pc, 32);
              if (lk == 0) sPart[p * NT + nt] = pc * rscale;
            }
            if constexpr (C::E4M3) {
              float am = fmaxf(fmaxf(fabsf(nv.x), fabsf(nv.y)), fmaxf(fabsf(nv.z), fabsf(nv.w)));
              am = fmaxf(am, __shfl_xor(am, 16));
              am = fmaxf(am, __shfl_xor(am, 32));
              if (lk == 0) sAmx[p * NT + nt] = am;
            }
          }
        }
        // the stores: the fp32 copy, the single bf16 copy, or the master (fp32 or bf16) and
        // the bf16 read copy (e4m3 codes after the row scale below)
#pragma unroll
        for (int i = 0; i < kMfmaTiles; ++i) {
          if (i < npt) {
            const size_t row = row0 + (pt0 + i) * 16 + li;
            const int col = nt * 16 + 4 * lk;
            if constexpr (COLD == NSSM_COLD_FP32)
              st_flush(acc[i], reinterpret_cast<f4*>(static_cast<float*>(a.cold) + row * NC + col));
            else if constexpr (SRC16)  // (acc holds bf16 values: this conversion is exact)
              st_flush(f32x4_to_bf16(acc[i].x, acc[i].y, acc[i].z, acc[i].w),
                        reinterpret_cast<u2v*>(static_cast<uint16_t*>(C::SEG ? a.cold : a.master) + blk16(row, col, NC)));
            else
              st_flush(acc[i], reinterpret_cast<f4*>(static_cast<float*>(a.master) + row * NC + col));
            if constexpr (COLD == NSSM_COLD_BF16)  // the read copy: RNE of the fp32 master
              st_flush(f32x4_to_bf16(acc[i].x, acc[i].y, acc[i].z, acc[i].w),
                        reinterpret_cast<u2v*>(static_cast<uint16_t*>(a.cold) + blk16(row, col, NC)));
          }
        }
        lds_barrier();  // partials and row maxima of this pass's tiles (and the next window)
        if constexpr (C::E4M3) {
#pragma unroll
          for (int i = 0; i < kMfmaTiles; ++i) {
            if (i < npt) {
              const int p = (pt0 + i) * 16 + li;
              const size_t row = row0 + p;
              float am = 0.f;
#pragma unroll
              for (int t2 = 0; t2 < NT; ++t2) am = fmaxf(am, sAmx[p * NT + t2]);
              const float sc = am / 448.0f + 1e-12f;  // scale/vllm_v4_patch.py:106-111
              const QDiv qd(sc);
              const f4 nv = acc[i];
              const uint32_t codes = f32x4_to_fp8(qd(nv.x), qd(nv.y), qd(nv.z), qd(nv.w));
              st_flush(codes, reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.cold) + row * NC + nt * 16 + 4 * lk));
              if (nt == 0 && lk == 0) a.scale[row] = sc;
              if constexpr (TF) {  // the readout of the new e4m3 copy
                float rd[4];
                fp8x4_to_f32(codes, rd);
                const f4 cq = *reinterpret_cast<const f4*>(sCq + nt * 16 + 4 * lk);
                float pc = rd[0] * cq.x;
                pc = fmaf(rd[1], cq.y, pc);
                pc = fmaf(rd[2], cq.z, pc);
                pc = fmaf(rd[3], cq.w, pc);
                pc += __shfl_xor(pc, 16);
                pc += __shfl_xor(pc, 32);
                if (lk == 0) sPart[p * NT + nt] = pc * sc;
              }
            }
          }
          // every wave has read the row maxima (the next item rewrites them) and, teacher-
          // forced, written its partials
          lds_barrier();
        }
        u0 += UPP;
      } while (u0 < nunit);
      // y += exp(glog) (stale cold readout); the next item's first barrier (pipelined:
      // its last, before this buffer of partials is written again) orders these reads
      if (tid < P) {
        float pc = 0.f;
#pragma unroll
        for (int t2 = 0; t2 < NT; ++t2) pc += sPart[tid * NT + t2];
        a.y[(size_t)it * P + tid] = fmaf(eg, pc, yv);
      }
      if (pipe) {
        // every wave has passed this item's last barrier, so its reads of window buffer buf
        // are done: the item after next is staged into it, and the next item's state tiles
        // (first pass) and y are loaded, all in flight during the next item's contraction
        const int kn1 = next_item(k + 1);
        if (kn1 < jn) {
          const int kn2 = next_item(kn1 + 1);
          if (kn2 < jn) stage_item(kn2, buf);
          load_tiles(kn1, 0);
          if (tid < P) yv = a.y[(size_t)sItem[kn1] * P + tid];
        }
        buf ^= 1;
      }
    }
  }
}

// join: full state -> tiers; one workgroup (4 waves) per (request, head). Rows go in
// units of 8 in the stream kernel's segment mapping (float4 per lane per 32-column
// segment): hot columns stored as they are, cold columns through cold_store (the fp32
// copy, or the fp32 master and the bf16 / e4m3 read copy with its row amax scale,
// scale/vllm_v4_patch.py:106-111).
template <int K, int COLD>
__global__ void __launch_bounds__(256) join_kernel(StepArgs a, const float* __restrict__ S,
                                                   const int32_t* __restrict__ phase) {
  using C = Cfg<K, COLD>;
  constexpr int HS = C::HS, CS = C::CS;
  const int bi = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
  if (slot < 0 || slot >= a.slots) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int q = lane & 7, rr = lane >> 3;
  for (int u = wave; u < (a.P >> 3); u += nw) {
    const int p = u * 8 + rr;
    const size_t row = ((size_t)slot * a.H + h) * a.P + p;
    const float* srow = S + (((size_t)bi * a.H + h) * a.P + p) * kN;
    const f4* src = reinterpret_cast<const f4*>(srow) + q;
    f4 hv[C::HSR];
    f2 hh = f2{0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < HS; ++s2) hv[s2] = ld_stream(src + 8 * s2);
    if constexpr (C::HH) hh = ld_stream(reinterpret_cast<const f2*>(srow + 32 * HS) + q);
    if constexpr (C::TIERED) {
      const float* crow = srow + K;  // the cold columns, in the segment mapping
      float v[C::CSR][4], vh[2] = {0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < CS; ++s2) {
        const f4 t = ld_stream(reinterpret_cast<const f4*>(crow) + q + 8 * s2);
        v[s2][0] = t.x; v[s2][1] = t.y; v[s2][2] = t.z; v[s2][3] = t.w;
      }
      if constexpr (C::CH) {
        const f2 t = ld_stream(reinterpret_cast<const f2*>(crow + 32 * CS) + q);
        vh[0] = t.x;
        vh[1] = t.y;
      }
      cold_store<COLD, CS, C::CH>(a, row, q, v, vh);
    }
    f4* hp = reinterpret_cast<f4*>(a.hot + row * K) + q;
#pragma unroll
    for (int s2 = 0; s2 < HS; ++s2) st_stream(hv[s2], hp + 8 * s2);
    if constexpr (C::HH) st_stream(hh, reinterpret_cast<f2*>(a.hot + row * K + 32 * HS) + q);
  }
  if (tid == 0) {
    const size_t o = (size_t)slot * a.H + h;
    a.t[o] = phase ? phase[bi] : 0;
    a.nv[o] = 0;
    a.glog[o] = 0.f;
  }
}

template <int K>
void launch_join(const StepArgs& a, int kind, const float* state, const int32_t* phase, unsigned grid,
                 hipStream_t st) {
  switch (kind) {
    case NSSM_COLD_FP32: hipLaunchKernelGGL((join_kernel<K, NSSM_COLD_FP32>), dim3(grid), dim3(256), 0, st, a, state, phase); break;
    case NSSM_COLD_BF16: hipLaunchKernelGGL((join_kernel<K, NSSM_COLD_BF16>), dim3(grid), dim3(256), 0, st, a, state, phase); break;
    case NSSM_COLD_FP8: hipLaunchKernelGGL((join_kernel<K, NSSM_COLD_FP8>), dim3(grid), dim3(256), 0, st, a, state, phase); break;
    case NSSM_COLD_BF16_SINGLE: hipLaunchKernelGGL((join_kernel<K, NSSM_COLD_BF16_SINGLE>), dim3(grid), dim3(256), 0, st, a, state, phase); break;
    case NSSM_COLD_FP8_BF16M: hipLaunchKernelGGL((join_kernel<K, NSSM_COLD_FP8_BF16M>), dim3(grid), dim3(256), 0, st, a, state, phase); break;
    default: hipLaunchKernelGGL((join_kernel<K, NSSM_COLD_NONE>), dim3(grid), dim3(256), 0, st, a, state, phase); break;
  }
}

// materialize: tiers -> exact full state; one workgroup per (request, head)
__global__ void materialize_kernel(StepArgs a, float* __restrict__ S, int K, int kind) {
  __shared__ float w[kMaxC + 1];
  __shared__ float lg[kMaxC];
  const int bi = blockIdx.x / a.H, h = blockIdx.x % a.H, g = h / a.HG;
  const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
  const int NC = kN - K, c = a.c;
  if (slot < 0 || slot >= a.slots) {
    for (int i = threadIdx.x; i < a.P * kN; i += blockDim.x)
      S[((size_t)bi * a.H + h) * a.P * kN + i] = __builtin_nanf("");
    return;
  }
  const size_t o = (size_t)slot * a.H + h;
  const int tcur = max(a.t[o], 0);
  const int nv = min(max(a.nv[o], 0), tcur % c);  // nv <= t % c, as prep clamps it
  const int t0 = tcur - nv;  // step count at the snapshot; pending token i sits at ring (t0 + i) % c
  const size_t rh = o * c;
  if ((int)threadIdx.x < nv) lg[threadIdx.x] = a.ring_dt[rh + (t0 + threadIdx.x) % c] * a.A[h];
  __syncthreads();
  if ((int)threadIdx.x < nv) {
    float suf = 0.f;
    for (int l = nv - 1; l > (int)threadIdx.x; --l) suf += lg[l];
    w[threadIdx.x] = expf(suf) * a.ring_dt[rh + (t0 + threadIdx.x) % c];
    if (threadIdx.x == 0) w[kMaxC] = expf(suf + lg[0]);
  }
  if (threadIdx.x == 0 && nv == 0) w[kMaxC] = 1.f;
  __syncthreads();
  const float dtot = w[kMaxC];
  const size_t rbg = ((size_t)slot * a.G + g) * c;
  for (int p = threadIdx.x; p < a.P; p += blockDim.x) {
    const size_t row = o * a.P + p;
    float* dst = S + (((size_t)bi * a.H + h) * a.P + p) * kN;
    for (int n = 0; n < K; ++n) dst[n] = a.hot[row * K + n];
    // the snapshot values: fp32 (the copy or the master) or bf16 (the single copy or the master)
    const bool m16 = kind == NSSM_COLD_BF16_SINGLE || kind == NSSM_COLD_FP8_BF16M;
    const void* cbase = kind == NSSM_COLD_FP32 || kind == NSSM_COLD_BF16_SINGLE ? a.cold : a.master;
    for (int n = 0; n < NC; ++n) {
      const float snap = m16 ? bf2f(static_cast<const uint16_t*>(cbase)[blk16(row, n, NC)])
                             : static_cast<const float*>(cbase)[row * NC + n];
      float v = dtot * snap;
      for (int i = 0; i < nv; ++i) {
        const int pos = (t0 + i) % c;
        const float u = w[i] * bf2f(a.ring_x[xring(a, o, pos, p)]);
        v = fmaf(u, a.ring_b[(rbg + pos) * NC + n], v);
      }
      dst[K + n] = v;
    }
  }
}

// fp8 dequant-matvec with per-(row, column) scale; one thread per (row, p)
__global__ void fp8_readout_kernel(const float* __restrict__ q, const uint8_t* __restrict__ s8,
                                   const float* __restrict__ scale, float* __restrict__ y, int rows, int nc,
                                   int pd) {
  const int r = blockIdx.y;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows || p >= pd) return;
  float acc = 0.f;
  const uint8_t* src = s8 + (size_t)r * nc * pd + p;
  for (int n = 0; n < nc; ++n) {
    const float qs = q[(size_t)r * nc + n] * scale[(size_t)r * nc + n];
    acc = fmaf(qs, nssm_e4m3fn_to_f32(src[(size_t)n * pd]), acc);
  }
  y[(size_t)r * pd + p] = acc;
}

// rotation of flat [T][G][N] bf16 vectors; one workgroup per (t, g), one thread per output m
// Duplicate and out-of-range slot ids of one call, on the device (one workgroup, so every
// thread uses the same tag): tag = state[0] + 1, never 0 (the owner words start at 0); request i
// exchanges (tag << 32 | i) into owner[slot] (64-bit vector atomics), and an old value with
// this call's tag (another request of the call holds the slot) sets bit 0 of state[1], an id
// outside [0, slots) bit 1; after every request, state[0] advances, so each call, graph
// replays included, has a tag of its own.
__global__ void __launch_bounds__(1024) check_slots_kernel(const int32_t* __restrict__ slot_ids, int b, int slots,
                                                           unsigned long long* owner, int32_t* state) {
  const uint32_t tag = (uint32_t)state[0] + 1u == 0u ? 1u : (uint32_t)state[0] + 1u;
  int bad = 0;
  for (int i = threadIdx.x; i < b; i += blockDim.x) {
    const int s = slot_ids[i];
    if (s < 0 || s >= slots) {
      bad |= 2;
      continue;
    }
    const unsigned long long old = atomicExch(owner + s, ((unsigned long long)tag << 32) | (uint32_t)i);
    if ((uint32_t)(old >> 32) == tag) bad |= 1;
  }
  if (bad) atomicOr(state + 1, bad);
  __syncthreads();  // every exchange of this call is done
  if (threadIdx.x == 0) state[0] = (int32_t)tag;
}

__global__ void rotate_kernel(const uint16_t* __restrict__ in, const float* __restrict__ R, float* __restrict__ out,
                              int G, int N) {
  extern __shared__ float sv[];
  const int tg = blockIdx.x, g = tg % G;
  for (int n = threadIdx.x; n < N; n += blockDim.x) sv[n] = bf2f(in[(size_t)tg * N + n]);
  __syncthreads();
  for (int m = threadIdx.x; m < N; m += blockDim.x) {
    const float* Rr = R + ((size_t)g * N + m) * N;
    float acc = 0.f;
    for (int n = 0; n < N; ++n) acc = fmaf(Rr[n], sv[n], acc);
    out[(size_t)tg * N + m] = acc;
  }
}

// ---------------------------------------------------------------------------
// conv prologue: causal depthwise conv1d update of one decode token + SiLU, one
// thread per (request, channel). DT: model dtype of hbc, state, weight, bias
// (0 fp32, 1 bf16; in bf16 the conv and the SiLU outputs are rounded to bf16, as
// torch computes them in that dtype).
constexpr int kMaxConvW = 8;

struct ConvArgs {
  const void* hbc;
  void* state;
  const void* w;
  const void* bias;
  const float* mask;
  uint16_t *x, *B, *C;
  int64_t hbc_stride;
  int32_t b, dim, W, I, GN;
};

template <int DT>
__device__ __forceinline__ float ld_dt(const void* p, size_t i) {
  if constexpr (DT == 0) return static_cast<const float*>(p)[i];
  else return bf2f(static_cast<const uint16_t*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void st_dt(void* p, size_t i, float v) {
  if constexpr (DT == 0) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = nssm_f32_to_bf16(v);  // v is a bf16 value: exact
}
template <int DT>
__device__ __forceinline__ float round_dt(float v) {
  if constexpr (DT == 0) return v;
  else return bf2f(nssm_f32_to_bf16(v));
}

template <int DT>
__global__ void __launch_bounds__(256) conv_update_kernel(ConvArgs a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.b * a.dim) return;
  const int r = (int)(i / a.dim), ch = (int)(i - (int64_t)r * a.dim);
  const int W = a.W;
  const size_t so = ((size_t)r * a.dim + ch) * W;
  const float xin = ld_dt<DT>(a.hbc, (size_t)r * a.hbc_stride + ch);
  float acc = a.bias ? ld_dt<DT>(a.bias, ch) : 0.f;
  if (W == 4) {  // the usual width: the state row and the weights as one vector each
    float s[4], w[4];
    if constexpr (DT == 0) {
      const f4 sv = *reinterpret_cast<const f4*>(static_cast<const float*>(a.state) + so);
      const f4 wv = *reinterpret_cast<const f4*>(static_cast<const float*>(a.w) + (size_t)ch * 4);
      s[0] = sv.x; s[1] = sv.y; s[2] = sv.z; s[3] = sv.w;
      w[0] = wv.x; w[1] = wv.y; w[2] = wv.z; w[3] = wv.w;
      *reinterpret_cast<f4*>(static_cast<float*>(a.state) + so) = f4{s[1], s[2], s[3], xin};
    } else {
      const u2v sv = *reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(a.state) + so);
      const u2v wv = *reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(a.w) + (size_t)ch * 4);
      s[0] = __uint_as_float(sv.x << 16); s[1] = __uint_as_float(sv.x & 0xffff0000u);
      s[2] = __uint_as_float(sv.y << 16); s[3] = __uint_as_float(sv.y & 0xffff0000u);
      w[0] = __uint_as_float(wv.x << 16); w[1] = __uint_as_float(wv.x & 0xffff0000u);
      w[2] = __uint_as_float(wv.y << 16); w[3] = __uint_as_float(wv.y & 0xffff0000u);
      const uint32_t xb = nssm_f32_to_bf16(xin);
      *reinterpret_cast<u2v*>(static_cast<uint16_t*>(a.state) + so) =
          u2v{(sv.x >> 16) | (sv.y << 16), (sv.y >> 16) | (xb << 16)};
    }
    acc = fmaf(s[1], w[0], acc);
    acc = fmaf(s[2], w[1], acc);
    acc = fmaf(s[3], w[2], acc);
    acc = fmaf(xin, w[3], acc);
  } else {
    float s[kMaxConvW], w[kMaxConvW];
#pragma unroll
    for (int k = 0; k < kMaxConvW; ++k) {
      if (k < W) {
        s[k] = ld_dt<DT>(a.state, so + k);
        w[k] = ld_dt<DT>(a.w, (size_t)ch * W + k);
      }
    }
    // shift in the new input; out = bias + sum_w state'[w] weight[w] (cross-correlation)
#pragma unroll
    for (int k = 0; k < kMaxConvW; ++k) {
      if (k < W) {
        const float v = k < W - 1 ? s[k + 1] : xin;
        st_dt<DT>(a.state, so + k, v);
        acc = fmaf(v, w[k], acc);
      }
    }
  }
  float u = round_dt<DT>(acc);
  u = round_dt<DT>(u / (1.f + expf(-u)));  // SiLU
  if (a.mask) u = round_dt<DT>(u * a.mask[r]);
  const uint16_t o = nssm_f32_to_bf16(u);
  if (ch < a.I) a.x[(size_t)r * a.I + ch] = o;
  else if (ch < a.I + a.GN) a.B[(size_t)r * a.GN + (ch - a.I)] = o;
  else a.C[(size_t)r * a.GN + (ch - a.I - a.GN)] = o;
}

// ---------------------------------------------------------------------------
// epilogue: gated RMSNorm of the mixer output, one workgroup (256 threads) per
// (request, group of gs channels); DT: model dtype of gate, weight and out.
constexpr int kNormThreads = 256;
constexpr int kNormPer = 8;  // channels per thread: gs <= 2048

struct NormArgs {
  const float* y;
  const void* gate;
  const void* w;
  void* out;
  int64_t gate_stride;
  int32_t I, gs;
  float eps;
};

template <int DT>
__global__ void __launch_bounds__(kNormThreads) gated_norm_kernel(NormArgs a) {
  __shared__ float sRed[kNormThreads / 64];
  const int ng = a.I / a.gs;
  const int r = blockIdx.x / ng, grp = blockIdx.x - r * ng;
  const int tid = threadIdx.x;
  const size_t c0 = (size_t)grp * a.gs;
  float v[kNormPer];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int i = tid + k * kNormThreads;
    v[k] = 0.f;
    if (i < a.gs) {
      const float yv = round_dt<DT>(a.y[(size_t)r * a.I + c0 + i]);  // y in the model dtype
      const float gv = ld_dt<DT>(a.gate, (size_t)r * a.gate_stride + c0 + i);
      v[k] = yv * (gv / (1.f + expf(-gv)));  // y * silu(gate), fp32
      ss = fmaf(v[k], v[k], ss);
    }
  }
  // group sum of squares: wave (DPP + cross-row shuffles), then across the waves
  ss += dpp<0xB1>(ss);
  ss += dpp<0x4E>(ss);
  ss += dpp<0x141>(ss);
  ss += __shfl_xor(ss, 8);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  if ((tid & 63) == 0) sRed[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += sRed[i];
  const float rs = 1.f / sqrtf(tot / (float)a.gs + a.eps);
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int i = tid + k * kNormThreads;
    if (i < a.gs) {
      const float o = ld_dt<DT>(a.w, c0 + i) * round_dt<DT>(v[k] * rs);
      if constexpr (DT == 0) static_cast<float*>(a.out)[(size_t)r * a.I + c0 + i] = o;
      else static_cast<uint16_t*>(a.out)[(size_t)r * a.I + c0 + i] = nssm_f32_to_bf16(o);
    }
  }
}

// One wave per (request, group) when gs is a multiple of 256 channels and the rows are
// 4-channel aligned: each lane takes 4 consecutive channels per 256 (y as 16 bytes, gate,
// weight and out as 8 bytes in bf16), issues the weight loads with the others, and the sum
// of squares is reduced inside the wave (no LDS, no barrier). Per channel the arithmetic
// is gated_norm_kernel's; the sum runs in another order. NB = gs / 256 is a template
// argument, so every block's loads go out together without run-time guards. (At the 9B
// shape, B = 256, 21 MB per launch: 7.3 us in graph replays whether the blocks' loads go
// out one block at a time or all at once, about 3.8 us of bandwidth and the rest a
// launch's fixed cost.)
constexpr int kNormWavePer = 8;  // 256-channel blocks per lane: gs <= 2048

template <int DT>
__device__ __forceinline__ void ld4_dt(const void* p, size_t i, float (&v)[4]) {
  if constexpr (DT == 0) {
    const f4 t = *reinterpret_cast<const f4*>(static_cast<const float*>(p) + i);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
    const u2v t = *reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(p) + i);
    v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
    v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
  }
}

template <int DT, int NB>
__global__ void __launch_bounds__(64) gated_norm_wave_kernel(NormArgs a) {
  const int ng = a.I / a.gs;
  const int r = blockIdx.x / ng, grp = blockIdx.x - r * ng;
  const int lane = threadIdx.x;
  const size_t c0 = (size_t)grp * a.gs + 4 * lane;
  float v[NB][4], w[NB][4];
  f4 yv[NB];
  float g[NB][4];
#pragma unroll
  for (int k = 0; k < NB; ++k) {  // every block's loads first
    const size_t c = c0 + 256 * k;
    yv[k] = *reinterpret_cast<const f4*>(a.y + (size_t)r * a.I + c);
    ld4_dt<DT>(a.gate, (size_t)r * a.gate_stride + c, g[k]);
    ld4_dt<DT>(a.w, c, w[k]);
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const float ys[4] = {yv[k].x, yv[k].y, yv[k].z, yv[k].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[k][e] = round_dt<DT>(ys[e]) * (g[k][e] / (1.f + expf(-g[k][e])));  // y * silu(gate), fp32
      ss = fmaf(v[k][e], v[k][e], ss);
    }
  }
  ss += dpp<0xB1>(ss);
  ss += dpp<0x4E>(ss);
  ss += dpp<0x141>(ss);
  ss += __shfl_xor(ss, 8);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  const float rs = 1.f / sqrtf(ss / (float)a.gs + a.eps);
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const size_t o = (size_t)r * a.I + c0 + 256 * k;
    float t[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = w[k][e] * round_dt<DT>(v[k][e] * rs);
    if constexpr (DT == 0) *reinterpret_cast<f4*>(static_cast<float*>(a.out) + o) = f4{t[0], t[1], t[2], t[3]};
    else
      *reinterpret_cast<u2v*>(static_cast<uint16_t*>(a.out) + o) =
          u2v{nssm_f32_to_bf16(t[0]) | ((uint32_t)nssm_f32_to_bf16(t[1]) << 16),
              nssm_f32_to_bf16(t[2]) | ((uint32_t)nssm_f32_to_bf16(t[3]) << 16)};
  }
}

// the wave kernel's instance for a dtype and a block count (host dispatch)
template <int DT, int NB>
struct NormWave {
  static constexpr auto fn = gated_norm_wave_kernel<DT, NB>;
};

// ---------------------------------------------------------------------------
// measurement aid: a plain streaming read or copy, the rate the state op's HBM traffic is
// compared with on the same device. Workgroup chunks of kProbeU x 256 float4 (each lane
// kProbeU 16-byte non-temporal loads 4 KiB apart, all issued before the first use),
// grid-stride over the chunks. Measured on MI355X over 2 GiB with 4096 workgroups: 6.8 TB/s
// read, 6.0 TB/s copy (read + write); 8 float4 per lane read at the same rate and copied at
// 5.7, 16 at 6.5 / 5.0, plain loads and stores at 6.2 / 5.4.
constexpr int kProbeU = 4;
constexpr int kProbeGrid = 4096;
constexpr int64_t kProbeChunk = kProbeU * 256 * 16;  // bytes per workgroup chunk

template <bool COPY>
__global__ void __launch_bounds__(256) stream_probe_kernel(const f4* __restrict__ a, f4* __restrict__ b,
                                                           int64_t nchunk) {
  f4 s = {0.f, 0.f, 0.f, 0.f};
  for (int64_t ch = blockIdx.x; ch < nchunk; ch += gridDim.x) {
    const int64_t o = ch * (kProbeU * 256) + threadIdx.x;
    f4 v[kProbeU];
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) v[u] = __builtin_nontemporal_load(a + o + u * 256);
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) {
      if constexpr (COPY) __builtin_nontemporal_store(v[u], b + o + u * 256);
      else s += v[u];
    }
  }
  // the read keeps its loads through a store no finite sum takes (b holds one float4)
  if constexpr (!COPY) {
    if (s.x + s.y + s.z + s.w == __builtin_inff()) b[0] = s;
  }
}

// ---------------------------------------------------------------------------
// host side
int g_units_override = 0;  // units (waves) per stream workgroup, 0 = automatic
#ifndef NSSM_FLUSH_PIPE
#define NSSM_FLUSH_PIPE 1
#endif
constexpr bool g_flush_pipe = NSSM_FLUSH_PIPE;  // stage the next flush item's window early when two fit
constexpr size_t kMaxLds = 64 * 1024;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }

int check_params(const nssm_layer_params* prm) {
  if (!prm || !prm->dt_bias || !prm->A || !prm->D) return NSSM_E_NULL;
  if (prm->N != kN || prm->H <= 0 || prm->G <= 0 || prm->H % prm->G || prm->H / prm->G > kMaxHG) return NSSM_E_DIMS;
  if (prm->P <= 0 || prm->P % 16 || prm->P > 256) return NSSM_E_DIMS;
  if (prm->R && !aligned16(prm->R)) return NSSM_E_ALIGN;
  return NSSM_OK;
}

int check_inputs(const nssm_step_inputs* in, const float* y) {
  if (!in || !in->x || !in->B || !in->C || !in->dt || !y) return NSSM_E_NULL;
  if (in->b < 0) return NSSM_E_DIMS;
  if (!aligned8(in->x)) return NSSM_E_ALIGN;
  return NSSM_OK;
}

int check_ws(const nssm_layer_params* prm, int b, int c, const void* ws, int64_t ws_bytes) {
  if (!ws) return NSSM_E_WORKSPACE;
  if (!aligned16(ws)) return NSSM_E_ALIGN;
  if (ws_bytes < (int64_t)(ws_floats(b, prm->H, prm->G, c) * sizeof(float))) return NSSM_E_WORKSPACE;
  return NSSM_OK;
}

// The no-allocation entry point's workspace: one fixed array per GPU (the code object's
// device global, created with the module on each device and held until the process ends).
// In host code `scratch` names a host-side stand-in: its device address on the current
// device comes from hipGetSymbolAddress, looked up once per device and kept in
// g_scratch_ptr; only that address is ever handed to a kernel.
static __device__ __align__(256) unsigned char scratch[NSSM_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, or nullptr when it cannot be found.
void* scratch_address() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (!p) {
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return nullptr;
    g_scratch_ptr[dev].store(q, std::memory_order_release);
    p = q;
  }
  return p;
}

// compute units of the current device (cached per device)
int cu_count() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}


// flush kernel LDS: a window buffer of fch tokens (B' fp32, x bf16, weights) and C'[K:]
// with its per-tile readout partials, two of each when pipelined, (+ e4m3 row maxima);
// the kernel's own lists take under 2 KB more
size_t flush_lds_bytes(int P, int K, int kind, int fch, bool pipe = false) {
  const int NC = kN - K, fa = flush_alloc_tokens(fch);
  const size_t tiles = (size_t)P * (NC / 16);
  const bool e4m3 = kind == NSSM_COLD_FP8 || kind == NSSM_COLD_FP8_BF16M;  // + row maxima
  const size_t buf = (size_t)flush_win_floats(fa, NC, P) + tiles;
  return ((pipe ? 2 : 1) * buf + (e4m3 ? tiles : 0)) * sizeof(float);
}
// LDS a flush workgroup may take: the device's per-workgroup limit, and a CU's LDS shared
// by the kFlushPerCU resident workgroups
size_t flush_lds_limit() {
  static size_t cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kMaxLds;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
      v = (int)kMaxLds;
    cache[dev] = std::min((size_t)v, (size_t)160 * 1024 / kFlushPerCU);
  }
  return cache[dev];
}
// whether two whole windows of c tokens fit (the flush kernel then stages each item's
// window during the previous item's contraction)
bool flush_pipe(int P, int K, int kind, int c) {
  return flush_lds_bytes(P, K, kind, (c + 3) & ~3, true) + sizeof(FlushList) + 256 <= flush_lds_limit();
}
// a kernel launched with more than 64 KB of dynamic LDS declares it first (once per
// kernel and device)
bool lds_opt_in(const void* fn) {
  static std::mutex mu;
  static std::set<std::pair<int, const void*>> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lk(mu);
  if (done.count({dev, fn})) return true;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)flush_lds_limit()) != hipSuccess)
    return false;
  done.insert({dev, fn});
  return true;
}
// window tokens the flush kernel stages at a time: the whole window (c rounded up to a
// multiple of 4) when its buffer (rounded up to 32 tokens, flush_alloc_tokens) fits, else
// the most whole 32-token steps that fit (0: none fit)
int flush_chunk(int P, int K, int kind, int c) {
  const size_t budget = kMaxLds - 2048;
  const size_t fixed = flush_lds_bytes(P, K, kind, 0);
  const size_t per_tok = (size_t)(kN - K + flush_x_stride(P) / 2 + 1) * sizeof(float);
  const int fit = fixed >= budget ? 0 : (int)((budget - fixed) / per_tok) & ~31;
  const int want = (c + 3) & ~3;
  return want <= fit ? want : fit;
}

// Longest window the stream kernel replays itself (VALU, window in LDS); longer ones go to
// the flush kernel (matrix cores). Measured on MI355X at the 9B shape, B = 256, 27 layers,
// ms per step, fused / split:
//   fp32 cold           c = 16  7.82 / 8.28   c = 32  8.58 / 7.94   c = 64 10.46 / 7.88
//   e4m3, bf16 master   c = 16  5.32 / 6.22   c = 32  5.62 / 5.53   c = 64  8.23 / 5.24
//   single bf16 copy    c = 16  6.25 / 6.73   c = 32  6.34 / 6.44   c = 64  8.81 / 6.31
int fuse_max_window(int kind) { return kind == NSSM_COLD_BF16_SINGLE ? kFusedMaxWindow : 16; }

// requests per prep workgroup: one head thread per (request, head)
int prep_requests(int HG) {
  const int r = kPrepThreads / HG;
  return r < 1 ? 1 : r > kPrepReq ? kPrepReq : r;
}

struct Launch {
  int uw;      // units (waves) per stream workgroup
  bool fused;  // flush windows replayed in the stream kernel
  size_t lds;  // its LDS bytes (the fused window)
};

// Stream launch shape, measured on MI355X at the 9B shape (B = 256, 27 layers, ms per
// step): fresh 1 unit per workgroup 11.95, 2 units 12.09; k_hot = 32 tiered 2 units (fp32
// cold c = 4 8.57, 1 unit 8.78; e4m3 over a bf16 master at B = 448 11.62, 1 unit 11.80).
int pick_launch(int P, int K, int c, Launch* out, int kind = NSSM_COLD_FP32) {
  const int RG = P / 8;
  const bool tiered = K < kN && kind != NSSM_COLD_NONE;
  int uw = tiered ? 2 : 1;
  if (g_units_override > 0) uw = g_units_override;
  if (uw > kMaxUnitsPerWg || RG % uw) return NSSM_E_TUNING;
  // (the fused kernels' exact-readout correction is sized for kFusedMaxWindow tokens)
  const bool fused = tiered && c <= fuse_max_window(kind) && c <= kFusedMaxWindow;
  const size_t lds = fused ? ((size_t)c * (kN - K) + (size_t)c * uw * 8) * sizeof(float) : 0;
  if (lds > kMaxLds || (tiered && !fused && flush_chunk(P, K, kind, c) < 4)) return NSSM_E_DIMS;
  out->uw = uw;
  out->fused = fused;
  out->lds = lds;
  return NSSM_OK;
}

void fill_common(StepArgs& a, const nssm_layer_params* prm, const nssm_step_inputs* in, float* y, void* ws) {
  a.x = in->x;
  a.Bm = in->B;
  a.Cm = in->C;
  a.dt_raw = in->dt;
  a.slot_ids = in->slot_ids;
  a.dt_bias = prm->dt_bias;
  a.A = prm->A;
  a.D = prm->D;
  a.R = prm->R;
  a.y = y;
  a.ws = static_cast<float*>(ws);
  a.b = in->b;
  a.H = prm->H;
  a.P = prm->P;
  a.G = prm->G;
  a.HG = prm->H / prm->G;
  a.dt_min = prm->dt_min;
}

int check_tier(const nssm_tier* tr, bool need_ring) {
  if (!tr) return NSSM_E_NULL;
  if (tr->cold_kind < NSSM_COLD_FP32 || tr->cold_kind > NSSM_COLD_FP8_BF16M) return NSSM_E_KIND;
  const bool cold = tr->cold_kind != NSSM_COLD_NONE;
  // (k_hot = 0: no hot tier, every column cold; its hot pointer is never read)
  if ((!tr->hot && tr->k_hot > 0) || !tr->t || !tr->nv || !tr->glog || (cold && !tr->cold)) return NSSM_E_NULL;
  if (cold && need_ring && (!tr->ring_x || !tr->ring_dt || !tr->ring_b)) return NSSM_E_NULL;
  const bool e4m3 = tr->cold_kind == NSSM_COLD_FP8 || tr->cold_kind == NSSM_COLD_FP8_BF16M;
  if ((tr->cold_kind == NSSM_COLD_BF16 || e4m3) && !tr->master) return NSSM_E_NULL;
  if (e4m3 && !tr->scale) return NSSM_E_NULL;
  if (tr->slots <= 0 || tr->c < 1 || tr->c > kMaxC) return NSSM_E_DIMS;
  if (tr->x_layout != NSSM_XRING_ROW && tr->x_layout != NSSM_XRING_UNIT) return NSSM_E_KIND;
  if (tr->k_hot != 0 && tr->k_hot != 16 && tr->k_hot != 32 && tr->k_hot != 64 && tr->k_hot != 96) return NSSM_E_DIMS;
  if (tr->k_hot == 0 && !cold) return NSSM_E_DIMS;
  if (!aligned16(tr->hot) || (cold && !aligned16(tr->cold)) || (tr->master && !aligned16(tr->master)))
    return NSSM_E_ALIGN;
  if (cold && need_ring && (!aligned16(tr->ring_x) || !aligned16(tr->ring_b))) return NSSM_E_ALIGN;
  return NSSM_OK;
}

void fill_tier(StepArgs& a, const nssm_tier* tr, int P) {
  a.hot = tr->hot;
  a.cold = tr->cold;
  a.scale = tr->scale;
  a.master = tr->master;
  a.ring_x = tr->ring_x;
  a.ring_dt = tr->ring_dt;
  a.ring_b = tr->ring_b;
  a.t = tr->t;
  a.nv = tr->nv;
  a.glog = tr->glog;
  a.slots = tr->slots;
  a.c = tr->c;
  a.K = tr->k_hot;
  const bool unit = tr->x_layout == NSSM_XRING_UNIT;
  a.xs_tok = unit ? 8 : P;
  a.xs_unit = unit ? 8 * tr->c : 8;
}

template <int K, int COLD>
int launch_pair(const StepArgs& a, const Launch& L, hipStream_t st) {
  constexpr bool TIERED = K < kN && COLD != NSSM_COLD_NONE;
  // k_hot = 0 (every column cold, the evaluation forward's mode "c1") serves the
  // teacher-forced readout only: the other stream and flush variants are not instantiated
  constexpr bool kTfOnly = K == 0;
  if constexpr (kTfOnly && !TIERED) return NSSM_E_KIND;
  if (kTfOnly && !a.tf && !a.lag) return NSSM_E_DIMS;
  if (a.b == 0) return NSSM_OK;
  StepArgs ap = a;
  ap.prb = prep_requests(a.HG);
  const unsigned pgrid = (unsigned)((a.b + ap.prb - 1) / ap.prb) * a.G;
  hipLaunchKernelGGL((prep_kernel<TIERED>), dim3(pgrid), dim3(kPrepThreads), 0, st, ap);
  const dim3 ugrid((unsigned)((size_t)a.b * a.H * (a.P / 8 / L.uw))), ublock(L.uw * 64);
  const float* hd_ro = Ws(a.ws, a.b, a.H, a.G, a.c).hd;  // the per-head scalars prep wrote
  if constexpr (TIERED) {
    const bool gated = a.hot_only || a.qgate_tau > 0.f;
    if (L.fused) {
      if (a.lag) {
        hipLaunchKernelGGL((unit_kernel_lag<K, COLD, true>), ugrid, ublock, L.lds, st, a, hd_ro);
      } else if constexpr (kTfOnly) {
        hipLaunchKernelGGL((unit_kernel_tf<K, COLD, true>), ugrid, ublock, L.lds, st, a, hd_ro);
      } else {
        if (a.exact) hipLaunchKernelGGL((unit_kernel<K, COLD, true, true>), ugrid, ublock, L.lds, st, a, hd_ro);
        else if (a.tf) hipLaunchKernelGGL((unit_kernel_tf<K, COLD, true>), ugrid, ublock, L.lds, st, a, hd_ro);
        else if (gated) hipLaunchKernelGGL((unit_kernel_gated<K, COLD, true>), ugrid, ublock, L.lds, st, a, hd_ro);
        else hipLaunchKernelGGL((unit_kernel<K, COLD, true, false>), ugrid, ublock, L.lds, st, a, hd_ro);
      }
      return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
    }
    if (a.lag) {
      hipLaunchKernelGGL((unit_kernel_lag<K, COLD, false>), ugrid, ublock, 0, st, a, hd_ro);
    } else if constexpr (kTfOnly) {
      hipLaunchKernelGGL((unit_kernel_tf<K, COLD, false>), ugrid, ublock, 0, st, a, hd_ro);
    } else {
      if (a.exact) hipLaunchKernelGGL((unit_kernel<K, COLD, false, true>), ugrid, ublock, 0, st, a, hd_ro);
      else if (a.tf) hipLaunchKernelGGL((unit_kernel_tf<K, COLD, false>), ugrid, ublock, 0, st, a, hd_ro);
      else if (gated) hipLaunchKernelGGL((unit_kernel_gated<K, COLD, false>), ugrid, ublock, 0, st, a, hd_ro);
      else hipLaunchKernelGGL((unit_kernel<K, COLD, false, false>), ugrid, ublock, 0, st, a, hd_ro);
    }
    // one resident round of workgroups: an empty launch dispatches no more than that,
    // and a full flush keeps every workgroup busy to the end
    const int items = a.b * a.H, cap = kFlushPerCU * cu_count();
    const int grid = items < cap ? items : cap;
    const size_t flds = flush_lds_bytes(a.P, K, COLD, a.fch, a.fpipe != 0);
    auto go = [&](auto kern) {
      if (flds > kMaxLds && !lds_opt_in(reinterpret_cast<const void*>(kern))) return NSSM_E_LAUNCH;
      hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kFlushWaves * 64), flds, st, a);
      return NSSM_OK;
    };
    int frc;
    if (a.lag) frc = go(flush_kernel<K, COLD, false, true>);
    else if constexpr (kTfOnly) frc = go(flush_kernel<K, COLD, true>);
    else frc = a.tf ? go(flush_kernel<K, COLD, true>) : go(flush_kernel<K, COLD, false>);
    if (frc) return frc;
  } else if constexpr (K == kN) {  // untiered
    hipLaunchKernelGGL(fresh_kernel, dim3((unsigned)((size_t)a.b * a.H * (a.P / 2))), dim3(64), 0, st, a, hd_ro);
  } else if constexpr (!kTfOnly) {  // hot tier only
    hipLaunchKernelGGL((unit_kernel<K, COLD, false, false>), ugrid, ublock, 0, st, a, hd_ro);
  }
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

template <int K>
int dispatch_kind(const StepArgs& a, int kind, const Launch& L, hipStream_t st) {
  switch (kind) {
    case NSSM_COLD_FP32: return launch_pair<K, NSSM_COLD_FP32>(a, L, st);
    case NSSM_COLD_BF16: return launch_pair<K, NSSM_COLD_BF16>(a, L, st);
    case NSSM_COLD_FP8: return launch_pair<K, NSSM_COLD_FP8>(a, L, st);
    case NSSM_COLD_NONE: return launch_pair<K, NSSM_COLD_NONE>(a, L, st);
    case NSSM_COLD_BF16_SINGLE: return launch_pair<K, NSSM_COLD_BF16_SINGLE>(a, L, st);
    case NSSM_COLD_FP8_BF16M: return launch_pair<K, NSSM_COLD_FP8_BF16M>(a, L, st);
  }
  return NSSM_E_KIND;
}

// The second read copy of a lagged readout: cold's dtype and layout (scale with the e4m3
// kinds), and the per-(slot, head) decay of the window between the two snapshots.
int check_lag(const nssm_tier* tr, const nssm_lag* lg) {
  if (!lg) return NSSM_E_NULL;
  const bool e4m3 = tr->cold_kind == NSSM_COLD_FP8 || tr->cold_kind == NSSM_COLD_FP8_BF16M;
  if (!lg->cold || !lg->wlog || (e4m3 && !lg->scale)) return NSSM_E_NULL;
  if (!aligned16(lg->cold)) return NSSM_E_ALIGN;
  return NSSM_OK;
}

// readout: 0 stale, 1 exact (rank-c correction), 2 teacher-forced, 3 lagged teacher-forced
int v4_step(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_step_inputs* in, float* y,
            void* workspace, int64_t workspace_bytes, void* stream, int readout, int hot_only = 0,
            float qgate_tau = 0.f, int64_t* qcounts = nullptr, const nssm_lag* lag = nullptr) {
  const int exact = readout == 1;
  int rc = check_params(prm);
  if (rc) return rc;
  if ((rc = check_inputs(in, y))) return rc;
  if ((rc = check_tier(tier, true))) return rc;
  if (readout && tier->cold_kind == NSSM_COLD_NONE) return NSSM_E_KIND;  // these readouts need the cold tier
  if (readout == 3 && (rc = check_lag(tier, lag))) return rc;
  if (tier->k_hot == 0 && readout < 2) return NSSM_E_DIMS;  // every column cold: teacher-forced only
  if (!(fabsf(qgate_tau) <= 3.0e38f)) return NSSM_E_DIMS;  // NaN or infinite threshold
  if (qcounts && (reinterpret_cast<uintptr_t>(qcounts) & 7)) return NSSM_E_ALIGN;
  if (!in->slot_ids && in->b > tier->slots) return NSSM_E_DIMS;
  if ((rc = check_ws(prm, in->b, tier->c, workspace, workspace_bytes))) return rc;
  StepArgs a = {};
  fill_common(a, prm, in, y, workspace);
  fill_tier(a, tier, prm->P);
  a.exact = exact;
  a.tf = readout == 2;
  if (readout == 3) {
    a.lag = 1;
    a.cold2 = lag->cold;
    a.scale2 = lag->scale;
    a.wlag = lag->wlog;
  }
  a.hot_only = hot_only != 0;
  a.qgate_tau = qgate_tau;
  a.qcounts = reinterpret_cast<unsigned long long*>(qcounts);
  Launch L;
  if ((rc = pick_launch(prm->P, tier->k_hot, tier->c, &L, tier->cold_kind))) return rc;
  a.split = !L.fused && tier->cold_kind != NSSM_COLD_NONE;
  a.fch = a.split ? flush_chunk(prm->P, tier->k_hot, tier->cold_kind, tier->c) : 0;
  a.fpipe = a.split && g_flush_pipe && flush_pipe(prm->P, tier->k_hot, tier->cold_kind, tier->c);
  if (a.fpipe) a.fch = (tier->c + 3) & ~3;
  a.fw = a.fpipe;
  hipStream_t st = (hipStream_t)stream;
  switch (tier->k_hot) {
    case 0: return dispatch_kind<0>(a, tier->cold_kind, L, st);
    case 16: return dispatch_kind<16>(a, tier->cold_kind, L, st);
    case 32: return dispatch_kind<32>(a, tier->cold_kind, L, st);
    case 64: return dispatch_kind<64>(a, tier->cold_kind, L, st);
    case 96: return dispatch_kind<96>(a, tier->cold_kind, L, st);
  }
  return NSSM_E_DIMS;
}


// Width 4, four consecutive channels per thread (dims, strides and pointers 4-channel
// aligned, as at the 9B shape): the 16 state values and 16 weights move as whole vectors,
// the input as one 8 / 16-byte load and the output as one 8-byte store, so a wave
// instruction carries 512 B of x / B / C instead of 128. Per channel the arithmetic is
// conv_update_kernel's, in the same order.
template <int DT>
__global__ void __launch_bounds__(256) conv_update4_kernel(ConvArgs a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 4-channel group
  const int dq = a.dim >> 2;
  if (i >= (int64_t)a.b * dq) return;
  const int r = (int)(i / dq), ch0 = 4 * (int)(i - (int64_t)r * dq);
  const size_t so = ((size_t)r * a.dim + ch0) * 4;  // first of the group's 16 state values
  // the bias and mask loads go out first, beside the state loads (one round trip in all)
  // (raw bits inside the branch, converted after it, so nothing waits for them there)
  f4 bf = f4{0.f, 0.f, 0.f, 0.f};  // fp32 bias
  u2v bh = u2v{0u, 0u};            // bf16 bias, channels 2 j, 2 j + 1 in word j
  float mk = 1.f;
  if (a.bias) {
    if constexpr (DT == 0) bf = *reinterpret_cast<const f4*>(static_cast<const float*>(a.bias) + ch0);
    else bh = *reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(a.bias) + ch0);
  }
  if (a.mask) mk = a.mask[r];
  float s[16], w[16], xin[4];
  uint32_t xraw[4];
  if constexpr (DT == 0) {
    const f4* sp = reinterpret_cast<const f4*>(static_cast<const float*>(a.state) + so);
    const f4* wp = reinterpret_cast<const f4*>(static_cast<const float*>(a.w) + (size_t)ch0 * 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f4 sv = sp[k], wv = wp[k];
      s[4 * k] = sv.x; s[4 * k + 1] = sv.y; s[4 * k + 2] = sv.z; s[4 * k + 3] = sv.w;
      w[4 * k] = wv.x; w[4 * k + 1] = wv.y; w[4 * k + 2] = wv.z; w[4 * k + 3] = wv.w;
    }
    const f4 xv = *reinterpret_cast<const f4*>(static_cast<const float*>(a.hbc) + (size_t)r * a.hbc_stride + ch0);
    xin[0] = xv.x; xin[1] = xv.y; xin[2] = xv.z; xin[3] = xv.w;
    f4* dp = reinterpret_cast<f4*>(static_cast<float*>(a.state) + so);
#pragma unroll
    for (int k = 0; k < 4; ++k) dp[k] = f4{s[4 * k + 1], s[4 * k + 2], s[4 * k + 3], xin[k]};
  } else {
    // bf16: state and weights as 8 words of two values each (word j: elements 2j, 2j+1)
    const u4v* sp = reinterpret_cast<const u4v*>(static_cast<const uint16_t*>(a.state) + so);
    const u4v* wp = reinterpret_cast<const u4v*>(static_cast<const uint16_t*>(a.w) + (size_t)ch0 * 4);
    const u4v s0 = sp[0], s1 = sp[1], w0 = wp[0], w1 = wp[1];
    const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s[2 * j] = __uint_as_float(sw[j] << 16); s[2 * j + 1] = __uint_as_float(sw[j] & 0xffff0000u);
      w[2 * j] = __uint_as_float(ww[j] << 16); w[2 * j + 1] = __uint_as_float(ww[j] & 0xffff0000u);
    }
    const u2v xv = *reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(a.hbc) + (size_t)r * a.hbc_stride + ch0);
    xraw[0] = xv.x & 0xffffu; xraw[1] = xv.x >> 16; xraw[2] = xv.y & 0xffffu; xraw[3] = xv.y >> 16;
#pragma unroll
    for (int k = 0; k < 4; ++k) xin[k] = __uint_as_float(xraw[k] << 16);
    // channel k's new row: (s1, s2), (s3, x) of its two words
    uint32_t nw[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      nw[2 * k] = (sw[2 * k] >> 16) | (sw[2 * k + 1] << 16);
      nw[2 * k + 1] = (sw[2 * k + 1] >> 16) | (xraw[k] << 16);
    }
    u4v* dp = reinterpret_cast<u4v*>(static_cast<uint16_t*>(a.state) + so);
    dp[0] = u4v{nw[0], nw[1], nw[2], nw[3]};
    dp[1] = u4v{nw[4], nw[5], nw[6], nw[7]};
  }
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t bw = k < 2 ? bh.x : bh.y;
    float acc = DT == 0 ? bf[k] : __uint_as_float(k & 1 ? bw & 0xffff0000u : bw << 16);  // the bias (0 without one)
    acc = fmaf(s[4 * k + 1], w[4 * k], acc);
    acc = fmaf(s[4 * k + 2], w[4 * k + 1], acc);
    acc = fmaf(s[4 * k + 3], w[4 * k + 2], acc);
    acc = fmaf(xin[k], w[4 * k + 3], acc);
    float u = round_dt<DT>(acc);
    u = round_dt<DT>(u / (1.f + expf(-u)));  // SiLU
    if (a.mask) u = round_dt<DT>(u * mk);
    o[k] = nssm_f32_to_bf16(u);
  }
  const u2v ov{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
  uint16_t* dst = ch0 < a.I ? a.x + (size_t)r * a.I + ch0
                  : ch0 < a.I + a.GN ? a.B + (size_t)r * a.GN + (ch0 - a.I)
                                     : a.C + (size_t)r * a.GN + (ch0 - a.I - a.GN);
  *reinterpret_cast<u2v*>(dst) = ov;
}

}  // namespace

// ---------------------------------------------------------------------------
extern "C" {

int nssm_abi_version(void) { return NSSM_ABI_VERSION; }

const char* nssm_strerror(int code) {
  switch (code) {
    case NSSM_OK: return "ok";
    case NSSM_E_NULL: return "a required pointer is NULL";
    case NSSM_E_DIMS: return "sizes out of the supported range";
    case NSSM_E_ALIGN: return "a pointer is not aligned as required (state, parameters, workspace, ring_b: 16 bytes; x, ring_x: 8)";
    case NSSM_E_KIND: return "unknown cold storage kind";
    case NSSM_E_LAUNCH: return "HIP kernel launch failed";
    case NSSM_E_TUNING: return "launch override does not fit the dimensions";
    case NSSM_E_WORKSPACE: return "workspace missing or smaller than nssm_step_workspace_bytes()";
    case NSSM_E_SCRATCH: return "the call needs more workspace than the library's fixed scratch array (NSSM_SCRATCH_BYTES) holds";
  }
  return "unknown nssm error";
}

int64_t nssm_step_workspace_bytes(int32_t b, int32_t H, int32_t G, int32_t N, int32_t c) {
  if (b < 0 || H <= 0 || G <= 0 || H % G || N != kN || c < 0 || c > kMaxC) return NSSM_E_DIMS;
  return (int64_t)(ws_floats(b, H, G, c) * sizeof(float));
}

int nssm_tier_sizes(int32_t slots, int32_t H, int32_t P, int32_t N, int32_t G, int32_t k_hot, int32_t c,
                    int32_t cold_kind, int64_t* sz) {
  if (!sz) return NSSM_E_NULL;
  if (slots <= 0 || H <= 0 || P <= 0 || N != kN || G <= 0 || k_hot < 0 || k_hot >= N || c < 1 || c > kMaxC)
    return NSSM_E_DIMS;
  if (cold_kind < NSSM_COLD_FP32 || cold_kind > NSSM_COLD_FP8_BF16M) return NSSM_E_KIND;
  if (k_hot == 0 && cold_kind == NSSM_COLD_NONE) return NSSM_E_DIMS;  // no column kept at all
  const int64_t rows = (int64_t)slots * H * P;
  const int64_t NC = N - k_hot;
  int64_t esz = 0, msz = 0;  // bytes per element of the cold copy and of the master
  switch (cold_kind) {
    case NSSM_COLD_FP32: esz = 4; break;
    case NSSM_COLD_BF16: esz = 2; msz = 4; break;
    case NSSM_COLD_FP8: esz = 1; msz = 4; break;
    case NSSM_COLD_BF16_SINGLE: esz = 2; break;
    case NSSM_COLD_FP8_BF16M: esz = 1; msz = 2; break;
  }
  const bool e4m3 = cold_kind == NSSM_COLD_FP8 || cold_kind == NSSM_COLD_FP8_BF16M;
  const int64_t ring = cold_kind == NSSM_COLD_NONE ? 0 : 1;
  sz[0] = rows * k_hot * 4;
  sz[1] = rows * NC * esz;
  sz[2] = e4m3 ? rows * 4 : 0;
  sz[3] = rows * NC * msz;
  sz[4] = ring * slots * H * c * P * 2;
  sz[5] = ring * slots * H * c * 4;
  sz[6] = ring * slots * G * c * NC * 4;
  sz[7] = (int64_t)slots * H * 4;
  sz[8] = (int64_t)slots * H * 4;
  sz[9] = (int64_t)slots * H * 4;
  return NSSM_OK;
}

int nssm_set_launch(int32_t units_per_wg) {
  if (units_per_wg < 0 || units_per_wg > kMaxUnitsPerWg) return NSSM_E_TUNING;
  g_units_override = units_per_wg;
  return NSSM_OK;
}

int nssm_fresh_step(const nssm_layer_params* prm, float* state, int32_t slots, const nssm_step_inputs* in,
                    float* y, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_params(prm);
  if (rc) return rc;
  if ((rc = check_inputs(in, y))) return rc;
  if (!state) return NSSM_E_NULL;
  if (!aligned16(state)) return NSSM_E_ALIGN;
  if (slots <= 0 || (!in->slot_ids && in->b > slots)) return NSSM_E_DIMS;
  if ((rc = check_ws(prm, in->b, 0, workspace, workspace_bytes))) return rc;
  StepArgs a = {};
  fill_common(a, prm, in, y, workspace);
  a.hot = state;
  a.slots = slots;
  a.c = 0;
  a.K = kN;
  Launch L;
  if ((rc = pick_launch(prm->P, kN, 0, &L))) return rc;
  return launch_pair<kN, NSSM_COLD_FP32>(a, L, (hipStream_t)stream);
}

int nssm_v4_step(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_step_inputs* in, float* y,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  return v4_step(prm, tier, in, y, workspace, workspace_bytes, stream, 0);
}

int nssm_v4_step_noalloc(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_step_inputs* in, float* y,
                         void* stream) {
  // the argument checks of nssm_v4_step first (they touch no device), then the size
  int rc = check_params(prm);
  if (rc) return rc;
  if ((rc = check_inputs(in, y))) return rc;
  if ((rc = check_tier(tier, true))) return rc;
  const size_t need = ws_floats(in->b, prm->H, prm->G, tier->c) * sizeof(float);
  if (need > (size_t)NSSM_SCRATCH_BYTES) return NSSM_E_SCRATCH;
  void* ws = scratch_address();
  if (!ws) return NSSM_E_LAUNCH;
  return v4_step(prm, tier, in, y, ws, (int64_t)NSSM_SCRATCH_BYTES, stream, 0);
}

int nssm_v4_step_exact(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_step_inputs* in, float* y,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  return v4_step(prm, tier, in, y, workspace, workspace_bytes, stream, 1);
}

int nssm_v4_step_teacher(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_step_inputs* in, float* y,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  return v4_step(prm, tier, in, y, workspace, workspace_bytes, stream, 2);
}

int nssm_v4_step_teacher_lagged(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_lag* lag,
                                const nssm_step_inputs* in, float* y, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  return v4_step(prm, tier, in, y, workspace, workspace_bytes, stream, 3, 0, 0.f, nullptr, lag);
}

int nssm_v4_step_gated(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_step_inputs* in, float* y,
                       void* workspace, int64_t workspace_bytes, int32_t hot_only, float qgate_tau,
                       int64_t* counts, void* stream) {
  return v4_step(prm, tier, in, y, workspace, workspace_bytes, stream, 0, hot_only, qgate_tau, counts);
}

int nssm_v4_join(const nssm_layer_params* prm, const nssm_tier* tier, const float* state, int32_t b,
                 const int32_t* slot_ids, const int32_t* phase, void* stream) {
  int rc = check_params(prm);
  if (rc) return rc;
  if ((rc = check_tier(tier, false))) return rc;
  if (!state) return NSSM_E_NULL;
  if (!aligned16(state)) return NSSM_E_ALIGN;
  if (b < 0 || (!slot_ids && b > tier->slots)) return NSSM_E_DIMS;
  if (b == 0) return NSSM_OK;
  StepArgs a = {};
  fill_tier(a, tier, prm->P);
  a.slot_ids = slot_ids;
  a.H = prm->H;
  a.P = prm->P;
  a.G = prm->G;
  a.HG = prm->H / prm->G;
  const unsigned grid = (unsigned)b * prm->H;
  switch (tier->k_hot) {
    case 0: launch_join<0>(a, tier->cold_kind, state, phase, grid, (hipStream_t)stream); break;
    case 16: launch_join<16>(a, tier->cold_kind, state, phase, grid, (hipStream_t)stream); break;
    case 32: launch_join<32>(a, tier->cold_kind, state, phase, grid, (hipStream_t)stream); break;
    case 64: launch_join<64>(a, tier->cold_kind, state, phase, grid, (hipStream_t)stream); break;
    case 96: launch_join<96>(a, tier->cold_kind, state, phase, grid, (hipStream_t)stream); break;
    default: return NSSM_E_DIMS;
  }
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

int nssm_v4_materialize(const nssm_layer_params* prm, const nssm_tier* tier, float* state_out, int32_t b,
                        const int32_t* slot_ids, void* stream) {
  int rc = check_params(prm);
  if (rc) return rc;
  if ((rc = check_tier(tier, true))) return rc;
  if (tier->cold_kind == NSSM_COLD_NONE) return NSSM_E_KIND;  // the cold columns were dropped
  if (!state_out) return NSSM_E_NULL;
  if (b < 0 || (!slot_ids && b > tier->slots)) return NSSM_E_DIMS;
  if (b == 0) return NSSM_OK;
  StepArgs a = {};
  fill_tier(a, tier, prm->P);
  a.slot_ids = slot_ids;
  a.A = prm->A;
  a.H = prm->H;
  a.P = prm->P;
  a.G = prm->G;
  a.HG = prm->H / prm->G;
  hipLaunchKernelGGL(materialize_kernel, dim3((unsigned)b * prm->H), dim3(128), 0, (hipStream_t)stream, a,
                     state_out, (int)tier->k_hot, (int)tier->cold_kind);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

int nssm_fp8_readout(const float* q, const uint8_t* s8, const float* scale, float* y, int32_t rows, int32_t nc,
                     int32_t pd, void* stream) {
  if (!q || !s8 || !scale || !y) return NSSM_E_NULL;
  if (rows < 0 || nc <= 0 || pd <= 0) return NSSM_E_DIMS;
  if (rows == 0) return NSSM_OK;
  dim3 grid((unsigned)((pd + 127) / 128), (unsigned)rows);
  hipLaunchKernelGGL(fp8_readout_kernel, grid, dim3(128), 0, (hipStream_t)stream, q, s8, scale, y, rows, nc, pd);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

int nssm_check_slots(const int32_t* slot_ids, int32_t b, int32_t slots, int64_t* owner, int32_t* state,
                     void* stream) {
  if (!slot_ids || !owner || !state) return NSSM_E_NULL;
  if (b < 0 || slots <= 0) return NSSM_E_DIMS;
  if (reinterpret_cast<uintptr_t>(owner) & 7) return NSSM_E_ALIGN;
  if (b == 0) return NSSM_OK;
  hipLaunchKernelGGL(check_slots_kernel, dim3(1), dim3(b < 1024 ? ((b + 63) & ~63) : 1024), 0, (hipStream_t)stream,
                     slot_ids, b, slots, reinterpret_cast<unsigned long long*>(owner), state);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

int nssm_rotate(const uint16_t* in, const float* R, float* out, int32_t T, int32_t G, int32_t N, void* stream) {
  if (!in || !R || !out) return NSSM_E_NULL;
  if (T < 0 || G <= 0 || N <= 0 || N > 1024) return NSSM_E_DIMS;
  if (T == 0) return NSSM_OK;
  hipLaunchKernelGGL(rotate_kernel, dim3((unsigned)T * G), dim3(128), N * sizeof(float), (hipStream_t)stream, in,
                     R, out, G, N);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

int nssm_conv_update(int32_t b, int32_t dim, int32_t width, int32_t dtype, const void* hbc, int64_t hbc_stride,
                     void* conv_state, const void* weight, const void* bias, const float* mask, int32_t I,
                     int32_t GN, uint16_t* x_out, uint16_t* B_out, uint16_t* C_out, void* stream) {
  if (!hbc || !conv_state || !weight || !x_out || !B_out || !C_out) return NSSM_E_NULL;
  if (b < 0 || width < 1 || width > kMaxConvW || I < 0 || GN < 0 || dim != I + 2 * GN || hbc_stride < dim)
    return NSSM_E_DIMS;
  // width 4 moves a state row and a weight row as one vector each
  if (width == 4 && (!(dtype == NSSM_DT_F32 ? aligned16(conv_state) && aligned16(weight)
                                             : aligned8(conv_state) && aligned8(weight))))
    return NSSM_E_ALIGN;
  if (dtype != NSSM_DT_F32 && dtype != NSSM_DT_BF16) return NSSM_E_KIND;
  if (b == 0 || dim == 0) return NSSM_OK;
  ConvArgs a{hbc, conv_state, weight, bias, mask, x_out, B_out, C_out, hbc_stride, b, dim, width, I, GN};
  const bool f32 = dtype == NSSM_DT_F32;
  const bool vec4 = width == 4 && I % 4 == 0 && GN % 4 == 0 && hbc_stride % 4 == 0 && aligned16(conv_state) &&
                    aligned16(weight) && (f32 ? aligned16(hbc) : aligned8(hbc)) && aligned8(x_out) &&
                    aligned8(B_out) && aligned8(C_out) && (!bias || (f32 ? aligned16(bias) : aligned8(bias)));
  if (vec4) {
    const unsigned grid4 = (unsigned)(((int64_t)b * (dim / 4) + 255) / 256);
    if (f32)
      hipLaunchKernelGGL(conv_update4_kernel<0>, dim3(grid4), dim3(256), 0, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL(conv_update4_kernel<1>, dim3(grid4), dim3(256), 0, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
  }
  const unsigned grid = (unsigned)(((int64_t)b * dim + 255) / 256);
  if (dtype == NSSM_DT_F32)
    hipLaunchKernelGGL(conv_update_kernel<0>, dim3(grid), dim3(256), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(conv_update_kernel<1>, dim3(grid), dim3(256), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

int nssm_gated_rmsnorm(int32_t b, int32_t I, int32_t gs, int32_t dtype, const float* y, const void* gate,
                       int64_t gate_stride, const void* weight, float eps, void* out, void* stream) {
  if (!y || !gate || !weight || !out) return NSSM_E_NULL;
  if (b < 0 || I <= 0 || gs <= 0 || I % gs || gs > kNormThreads * kNormPer || gate_stride < I) return NSSM_E_DIMS;
  if (dtype != NSSM_DT_F32 && dtype != NSSM_DT_BF16) return NSSM_E_KIND;
  if (b == 0) return NSSM_OK;
  NormArgs a{y, gate, weight, out, gate_stride, I, gs, eps};
  const dim3 grid((unsigned)b * (unsigned)(I / gs));
  // the wave kernel's 4-channel accesses: 16 bytes of y, 4 elements of the model dtype
  const uintptr_t va = dtype == NSSM_DT_F32 ? 15u : 7u;
  if (gs % 256 == 0 && gs / 256 <= kNormWavePer && gate_stride % 4 == 0 && aligned16(y) &&
      !((uintptr_t)gate & va) && !((uintptr_t)weight & va) && !((uintptr_t)out & va)) {
    const bool f32 = dtype == NSSM_DT_F32;
    auto go = [&](auto k0, auto k1) {
      if (f32) hipLaunchKernelGGL(decltype(k0)::fn, grid, dim3(64), 0, (hipStream_t)stream, a);
      else hipLaunchKernelGGL(decltype(k1)::fn, grid, dim3(64), 0, (hipStream_t)stream, a);
    };
    switch (gs / 256) {
      case 1: go(NormWave<0, 1>{}, NormWave<1, 1>{}); break;
      case 2: go(NormWave<0, 2>{}, NormWave<1, 2>{}); break;
      case 3: go(NormWave<0, 3>{}, NormWave<1, 3>{}); break;
      case 4: go(NormWave<0, 4>{}, NormWave<1, 4>{}); break;
      case 5: go(NormWave<0, 5>{}, NormWave<1, 5>{}); break;
      case 6: go(NormWave<0, 6>{}, NormWave<1, 6>{}); break;
      case 7: go(NormWave<0, 7>{}, NormWave<1, 7>{}); break;
      default: go(NormWave<0, 8>{}, NormWave<1, 8>{}); break;
    }
    return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
  }
  if (dtype == NSSM_DT_F32)
    hipLaunchKernelGGL(gated_norm_kernel<0>, grid, dim3(kNormThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(gated_norm_kernel<1>, grid, dim3(kNormThreads), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

int nssm_stream_probe(const void* src, void* dst, int64_t bytes, int32_t mode, void* stream) {
  if (!src || !dst) return NSSM_E_NULL;
  if (bytes <= 0 || bytes % kProbeChunk || (mode != 0 && mode != 1)) return NSSM_E_DIMS;
  if (!aligned16(src) || !aligned16(dst)) return NSSM_E_ALIGN;
  const f4* a = static_cast<const f4*>(src);
  f4* b = static_cast<f4*>(dst);
  if (mode == 0)
    hipLaunchKernelGGL(stream_probe_kernel<false>, dim3(kProbeGrid), dim3(256), 0, (hipStream_t)stream, a, b,
                       bytes / kProbeChunk);
  else
    hipLaunchKernelGGL(stream_probe_kernel<true>, dim3(kProbeGrid), dim3(256), 0, (hipStream_t)stream, a, b,
                       bytes / kProbeChunk);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

void nssm_host_f32_to_e4m3fn(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = nssm_f32_to_e4m3fn(in[i]);
}
void nssm_host_e4m3fn_to_f32(const uint8_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = nssm_e4m3fn_to_f32(in[i]);
}
void nssm_host_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = nssm_f32_to_bf16(in[i]);
}

}  // extern "C"
