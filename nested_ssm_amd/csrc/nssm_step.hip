// gfx950 kernels for the Mamba2 decode-step recurrent-state update with
// nested hot/cold tiering, and the C ABI declared in include/nssm.h.
//
// One layer-token is two launches on the caller's stream:
//
//  prep    one workgroup per (request, group). Rotates B and C once
//          (B' = R_g B, C' = R_g C, fp32) into the workspace, computes each
//          head's dt, decay, the stale-read factor exp(glog), the flush flag
//          and, at a flush, the decay weights of the buffered window; updates
//          t, nv, glog; appends this token (x, dt, B' cold columns) to the ring
//          at position t % c. A flush token sits at c-1, so a flush window is
//          always ring positions [c-m, c).
//  stream  one workgroup per (request, head block): streams the state rows.
//          A "unit" is 8 consecutive headdim rows p of one head. In a unit,
//          lane l owns row p0 + (l >> 3) and, in every 32-column segment s, the
//          four columns 32 s + 4 (l & 7) .. +3. One dwordx4 per lane per
//          segment moves 8 rows x 128 B = 1 KB per wave instruction; the C.h
//          readout of a row is a sum over its 8 lanes (three DPP steps).
//          Hot columns [0, K) are read and written every token; cold columns
//          [K, N) are only read, except at the request's flush token, when the
//          workgroup replays the staged window into them.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/nssm.h"
#include "nssm_formats.h"

namespace {

constexpr int kN = 128;  // d_state handled by these kernels
constexpr int kMaxC = 64;
constexpr int kMaxWaves = 8;
constexpr int kMfmaTiles = 8;  // 16 x 16 flush-contraction tiles a wave keeps in registers

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

struct StepArgs {
  // tier state (fresh: hot is the full state, the rest NULL)
  float* hot;
  void* cold;
  float* scale;
  float* master;
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
  int32_t b, slots, H, P, G, HG, c, K, hpw, nhb;
  float dt_min;
};

// Workspace carve-up for b requests (floats): rotated B and C [b][G][N] each,
// per-head scalars [b][H][HD_STRIDE], flush weights [b][H][c].
enum { HD_DT = 0, HD_A, HD_DECAY, HD_EG, HD_D, HD_FLUSH, HD_DTOT, HD_M, HD_POS, HD_STRIDE = 12 };
struct Ws {
  float *B, *C, *hd, *w;
  __host__ __device__ Ws(float* base, int b, int H, int G, int c) {
    B = base;
    C = B + (size_t)b * G * kN;
    hd = C + (size_t)b * G * kN;
    w = hd + (size_t)b * H * HD_STRIDE;
  }
};
size_t ws_floats(int b, int H, int G, int c) { return (size_t)b * (2 * G * kN + H * HD_STRIDE + H * c); }

__device__ __forceinline__ float bf2f(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// DPP controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror (lane i <-> 7-i within 8) = 0x141, row_mirror (within 16) = 0x140.
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
__device__ __forceinline__ float sum32(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v += __shfl_xor(v, 16);
  return v;
}

__device__ __forceinline__ float softplus_f(float v) { return v > 20.f ? v : log1pf(expf(v)); }

// Streaming access to the state: non-temporal (the state is touched once per
// token and is far larger than L2 and the MALL) unless built otherwise.
#ifndef NSSM_NT_LOAD
#define NSSM_NT_LOAD 1
#endif
#ifndef NSSM_NT_STORE
#define NSSM_NT_STORE 1
#endif
// units (8-row blocks) whose loads a wave keeps in flight together
#ifndef NSSM_UNROLL
#define NSSM_UNROLL 2
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

// ---------------------------------------------------------------------------
// prep: one workgroup (256 threads = 4 waves) per (request, group). Latency
// bound: every independent global load is issued before the first barrier.
constexpr int kPrepThreads = 256;

template <bool TIERED>
__global__ void __launch_bounds__(kPrepThreads) prep_kernel(StepArgs a) {
  constexpr int NW = kPrepThreads / 64;
  constexpr int ROWS = kN / (2 * NW);  // rows of R per half-wave
  constexpr int RB = ROWS / 2;         // rows per batch in flight
  __shared__ float sBraw[kN], sCraw[kN], sBr[kN];
  __shared__ int sPos, sFlush;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x % a.G, bi = blockIdx.x / a.G;
  const int H = a.H, HG = a.HG, c = a.c;
  const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
  if (slot < 0 || slot >= a.slots) return;  // the stream kernel writes NaN rows for it
  const Ws ws(a.ws, a.b, H, a.G, c);
  const size_t bgo = ((size_t)bi * a.G + g) * kN;
  const int hw = lane >> 5, hl = lane & 31;
  const float* __restrict__ Rg = a.R ? a.R + (size_t)g * kN * kN : nullptr;

  // 1. independent loads: first batch of R rows, B and C, the head's inputs
  f4 r[RB];
  if (Rg) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
      r[i] = *reinterpret_cast<const f4*>(Rg + (size_t)(2 * wave + hw + 2 * NW * i) * kN + 4 * hl);
  }
  if (tid < kN) {
    sBraw[tid] = bf2f(a.Bm[bgo + tid]);
    sCraw[tid] = bf2f(a.Cm[bgo + tid]);
  }
  const bool head_thread = tid < HG;
  const int h = g * HG + tid;
  const size_t o = (size_t)slot * H + h;
  float draw = 0.f, dtb = 0.f, Ah = 0.f, Dh = 0.f, gl = 0.f;
  int tt = 0, nvv = 0;
  if (head_thread) {
    draw = bf2f(a.dt_raw[(size_t)bi * H + h]);
    dtb = a.dt_bias[h];
    Ah = a.A[h];
    Dh = a.D[h];
    if constexpr (TIERED) {
      tt = a.t[o];
      nvv = a.nv[o];
      gl = a.glog[o];
    }
  }
  __syncthreads();

  // 2. rotation: a half-wave per row of R (both halves see the same rows
  // count, so every reduction runs with all lanes active)
  if (Rg) {
    const f4 bv = *reinterpret_cast<const f4*>(sBraw + 4 * hl);
    const f4 cv = *reinterpret_cast<const f4*>(sCraw + 4 * hl);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (half == 1) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
          r[i] = *reinterpret_cast<const f4*>(Rg + (size_t)(2 * wave + hw + 2 * NW * (RB + i)) * kN + 4 * hl);
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int mrow = 2 * wave + hw + 2 * NW * (half * RB + i);
        float db = r[i].x * bv.x;
        db = fmaf(r[i].y, bv.y, db);
        db = fmaf(r[i].z, bv.z, db);
        db = fmaf(r[i].w, bv.w, db);
        float dc = r[i].x * cv.x;
        dc = fmaf(r[i].y, cv.y, dc);
        dc = fmaf(r[i].z, cv.z, dc);
        dc = fmaf(r[i].w, cv.w, dc);
        db = sum32(db);
        dc = sum32(dc);
        if (hl == 0) {
          sBr[mrow] = db;
          ws.B[bgo + mrow] = db;
          ws.C[bgo + mrow] = dc;
        }
      }
    }
  } else if (tid < kN) {
    sBr[tid] = sBraw[tid];
    ws.B[bgo + tid] = sBraw[tid];
    ws.C[bgo + tid] = sCraw[tid];
  }

  // 3. per-head scalars and bookkeeping: one thread per head of the group
  if (head_thread) {
    float dt = softplus_f(draw + dtb);
    if (a.dt_min > 0.f) dt = fmaxf(dt, a.dt_min);
    const float av = dt * Ah;
    float* __restrict__ hd = ws.hd + ((size_t)bi * H + h) * HD_STRIDE;
    hd[HD_DT] = dt;
    hd[HD_A] = av;
    hd[HD_DECAY] = expf(av);
    hd[HD_D] = Dh;
    if constexpr (TIERED) {
      // t >= 0 and 0 <= nv < c hold for every tier these kernels write; the
      // clamps keep ring indexing inside the buffers even for a corrupted phase
      tt = max(tt, 0);
      nvv = min(max(nvv, 0), c - 1);
      const int pos = tt % c;
      const bool flush = (tt + 1) % c == 0;  // then pos == c - 1
      hd[HD_EG] = expf(gl);
      hd[HD_FLUSH] = flush ? 1.f : 0.f;
      hd[HD_POS] = (float)pos;
      if (flush) {
        // window = the nv buffered tokens at ring [c-m, c-1) and this one:
        // w_i = exp(sum_{l>i} a_l) dt_i, total decay exp(sum_l a_l)
        const int m = nvv + 1;
        const float* __restrict__ rdt = a.ring_dt + o * c + (c - m);
        float* __restrict__ w = ws.w + ((size_t)bi * H + h) * c;
        float suf = 0.f;
        for (int i = m - 1; i >= 0; --i) {
          const float dti = i == m - 1 ? dt : rdt[i];
          w[i] = expf(suf) * dti;
          suf += dti * Ah;
        }
        hd[HD_DTOT] = expf(suf);
        hd[HD_M] = (float)m;
        a.nv[o] = 0;
        a.glog[o] = 0.f;
      } else {
        hd[HD_DTOT] = 1.f;
        hd[HD_M] = 0.f;
        a.ring_dt[o * c + pos] = dt;
        a.nv[o] = nvv + 1;
        a.glog[o] = gl + av;
      }
      a.t[o] = tt + 1;
      if (tid == 0) {
        sPos = pos;
        sFlush = flush;
      }
    } else {
      hd[HD_EG] = 0.f;
      hd[HD_FLUSH] = 0.f;
      hd[HD_DTOT] = 1.f;
      hd[HD_M] = 0.f;
      hd[HD_POS] = 0.f;
    }
  }

  // 4. ring append of the rotated B cold columns (tokens that do not flush;
  // a flush token's columns are read from the workspace). x goes to the ring
  // from the stream kernel.
  if constexpr (TIERED) {
    __syncthreads();  // sPos, sFlush, sBr
    if (!sFlush) {
      const int NC = kN - a.K;
      const size_t rb = (((size_t)slot * a.G + g) * c + sPos) * NC;
      for (int n = tid; n < NC; n += kPrepThreads) a.ring_b[rb + n] = sBr[a.K + n];
    }
  }
}

// ---------------------------------------------------------------------------
// stream: raw registers of one unit for one lane: HS hot float4 and CS cold
// segments (float4 / 4 x bf16 / 4 x e4m3 by storage kind).
template <int K, int COLD>
struct UnitRaw {
  static constexpr int HS = K / 32;
  static constexpr int CS = COLD == NSSM_COLD_NONE ? 0 : (kN - K) / 32;
  static constexpr int CSR = CS > 0 ? CS : 1;
  f4 hv[HS];
  f4 cf[COLD == NSSM_COLD_FP32 ? CSR : 1];
  u2v cb[COLD == NSSM_COLD_BF16 ? CSR : 1];
  uint32_t c8[COLD == NSSM_COLD_FP8 ? CSR : 1];
  float sc;
  float xp;
  uint16_t xraw;
};

template <int K, int COLD>
__device__ __forceinline__ void unit_load(const StepArgs& a, size_t row, size_t xrow, int q, UnitRaw<K, COLD>& d) {
  constexpr int HS = K / 32, CS = UnitRaw<K, COLD>::CS, NC = kN - K;
  const f4* hp = reinterpret_cast<const f4*>(a.hot + row * K) + q;
#pragma unroll
  for (int s = 0; s < HS; ++s) d.hv[s] = ld_stream(hp + 8 * s);
  if constexpr (CS > 0) {
    if constexpr (COLD == NSSM_COLD_FP32) {
      const f4* p = reinterpret_cast<const f4*>(static_cast<const float*>(a.cold) + row * NC) + q;
#pragma unroll
      for (int s = 0; s < CS; ++s) d.cf[s] = ld_stream(p + 8 * s);
    } else if constexpr (COLD == NSSM_COLD_BF16) {
      const u2v* p = reinterpret_cast<const u2v*>(static_cast<const uint16_t*>(a.cold) + row * NC) + q;
#pragma unroll
      for (int s = 0; s < CS; ++s) d.cb[s] = ld_stream(p + 8 * s);
    } else {
      const uint32_t* p = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(a.cold) + row * NC) + q;
#pragma unroll
      for (int s = 0; s < CS; ++s) d.c8[s] = ld_stream(p + 8 * s);
      d.sc = a.scale[row];
    }
  }
  d.xraw = a.x[xrow];
  d.xp = bf2f(d.xraw);
}

// read-copy values the readout sees
template <int K, int COLD>
__device__ __forceinline__ void cold_decode(const UnitRaw<K, COLD>& d, float (&v)[UnitRaw<K, COLD>::CSR][4]) {
  constexpr int CS = UnitRaw<K, COLD>::CS;
#pragma unroll
  for (int s = 0; s < CS; ++s) {
    if constexpr (COLD == NSSM_COLD_FP32) {
      v[s][0] = d.cf[s].x; v[s][1] = d.cf[s].y; v[s][2] = d.cf[s].z; v[s][3] = d.cf[s].w;
    } else if constexpr (COLD == NSSM_COLD_BF16) {
      v[s][0] = __uint_as_float(d.cb[s].x << 16);
      v[s][1] = __uint_as_float(d.cb[s].x & 0xffff0000u);
      v[s][2] = __uint_as_float(d.cb[s].y << 16);
      v[s][3] = __uint_as_float(d.cb[s].y & 0xffff0000u);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[s][e] = nssm_e4m3fn_to_f32((uint8_t)(d.c8[s] >> (8 * e))) * d.sc;
    }
  }
}

// Write the new exact cold values of one row: fp32 copy, or master + read copy.
template <int COLD, int CS>
__device__ __forceinline__ void cold_store(const StepArgs& a, size_t row, int q, const float (&v)[CS][4]) {
  constexpr int NC = CS * 32;
  if constexpr (COLD == NSSM_COLD_FP32) {
    f4* p = reinterpret_cast<f4*>(static_cast<float*>(a.cold) + row * NC) + q;
#pragma unroll
    for (int s = 0; s < CS; ++s) st_stream(f4{v[s][0], v[s][1], v[s][2], v[s][3]}, p + 8 * s);
  } else {
    f4* pm = reinterpret_cast<f4*>(a.master + row * NC) + q;
#pragma unroll
    for (int s = 0; s < CS; ++s) st_stream(f4{v[s][0], v[s][1], v[s][2], v[s][3]}, pm + 8 * s);
    if constexpr (COLD == NSSM_COLD_BF16) {
      u2v* p = reinterpret_cast<u2v*>(static_cast<uint16_t*>(a.cold) + row * NC) + q;
#pragma unroll
      for (int s = 0; s < CS; ++s) {
        u2v t;
        t.x = (uint32_t)nssm_f32_to_bf16(v[s][0]) | ((uint32_t)nssm_f32_to_bf16(v[s][1]) << 16);
        t.y = (uint32_t)nssm_f32_to_bf16(v[s][2]) | ((uint32_t)nssm_f32_to_bf16(v[s][3]) << 16);
        st_stream(t, p + 8 * s);
      }
    } else {  // FP8 with per-row amax scale, as scale/vllm_v4_patch.py:106-111
      float am = 0.f;
#pragma unroll
      for (int s = 0; s < CS; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) am = fmaxf(am, fabsf(v[s][e]));
      am = max8(am);
      const float sc = am / 448.0f + 1e-12f;
      uint32_t* p = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.cold) + row * NC) + q;
#pragma unroll
      for (int s = 0; s < CS; ++s) {
        uint32_t t = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) t |= (uint32_t)nssm_f32_to_e4m3fn(v[s][e] / sc) << (8 * e);
        st_stream(t, p + 8 * s);
      }
      if (q == 0) a.scale[row] = sc;
    }
  }
}

// Compute and store one unit (8 rows of head h) from its raw registers. FLUSH
// selects the replay of the staged window (sU [m][P] of this head, sBc [m][NC]).
template <int K, int COLD, bool FLUSH>
__device__ __forceinline__ void unit_compute(const StepArgs& a, size_t row, size_t yrow, int p, int q,
                                             UnitRaw<K, COLD>& d, uint16_t* rx, const float* __restrict__ hd,
                                             const float (&Bh)[K / 32][4], const float (&Ch)[K / 32][4],
                                             const float (&Cc)[UnitRaw<K, COLD>::CSR][4], const float* sU,
                                             const float* sBc, int m, const float* dS = nullptr) {
  constexpr int HS = K / 32;
  constexpr int NC = kN - K;
  constexpr int CS = UnitRaw<K, COLD>::CS;
  constexpr int CSR = UnitRaw<K, COLD>::CSR;
  const int P = a.P;
  const float xp = d.xp;
  const float uu = hd[HD_DT] * xp;
  const float dec = hd[HD_DECAY];
  float ph = 0.f;
  f4* hp = reinterpret_cast<f4*>(a.hot + row * K) + q;
#pragma unroll
  for (int s = 0; s < HS; ++s) {
    f4 v = d.hv[s];
    v.x = fmaf(v.x, dec, uu * Bh[s][0]);
    v.y = fmaf(v.y, dec, uu * Bh[s][1]);
    v.z = fmaf(v.z, dec, uu * Bh[s][2]);
    v.w = fmaf(v.w, dec, uu * Bh[s][3]);
    ph = fmaf(v.x, Ch[s][0], ph);
    ph = fmaf(v.y, Ch[s][1], ph);
    ph = fmaf(v.z, Ch[s][2], ph);
    ph = fmaf(v.w, Ch[s][3], ph);
    st_stream(v, hp + 8 * s);
  }

  float part = ph;
  if constexpr (CS > 0) {
    float cv[CSR][4];
    cold_decode<K, COLD>(d, cv);
    float pc = 0.f;
#pragma unroll
    for (int s = 0; s < CS; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) pc = fmaf(cv[s][e], Cc[s][e], pc);
    part = fmaf(hd[HD_EG], pc, ph);

    if constexpr (FLUSH) {
      // exact cold state at this token: decayed snapshot + decayed replay of
      // the window (buffered tokens and this one), scale/v4_fused_decode.py:76-85
      float nvv[CS][4];
      if constexpr (COLD == NSSM_COLD_FP32) {
#pragma unroll
        for (int s = 0; s < CS; ++s)
#pragma unroll
          for (int e = 0; e < 4; ++e) nvv[s][e] = cv[s][e];
      } else {
        const f4* pm = reinterpret_cast<const f4*>(a.master + row * NC) + q;
#pragma unroll
        for (int s = 0; s < CS; ++s) {
          const f4 t = ld_stream(pm + 8 * s);
          nvv[s][0] = t.x; nvv[s][1] = t.y; nvv[s][2] = t.z; nvv[s][3] = t.w;
        }
      }
      const float dtot = hd[HD_DTOT];
#pragma unroll
      for (int s = 0; s < CS; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) nvv[s][e] *= dtot;
      if (dS) {  // window contraction done on the matrix cores, rows of stride NC + 4
        const float* dr = dS + p * (NC + 4) + 4 * q;
#pragma unroll
        for (int s = 0; s < CS; ++s) {
          const f4 dd = *reinterpret_cast<const f4*>(dr + 32 * s);
          nvv[s][0] += dd.x;
          nvv[s][1] += dd.y;
          nvv[s][2] += dd.z;
          nvv[s][3] += dd.w;
        }
      } else {
        for (int i = 0; i < m; ++i) {
          const float coef = sU[i * P + p];
          const float* bc = sBc + i * NC + 4 * q;
#pragma unroll
          for (int s = 0; s < CS; ++s) {
            const f4 bb = *reinterpret_cast<const f4*>(bc + 32 * s);
            nvv[s][0] = fmaf(coef, bb.x, nvv[s][0]);
            nvv[s][1] = fmaf(coef, bb.y, nvv[s][1]);
            nvv[s][2] = fmaf(coef, bb.z, nvv[s][2]);
            nvv[s][3] = fmaf(coef, bb.w, nvv[s][3]);
          }
        }
      }
      cold_store<COLD, CS>(a, row, q, nvv);
    }
  }
  part = sum8(part);
  if (q == 0) {
    a.y[yrow] = fmaf(hd[HD_D], xp, part);
    if (rx) rx[p] = d.xraw;  // ring append of x (tokens that do not flush)
  }
}

// one workgroup per (request, block of hpw heads of one group)
template <int K, int COLD>
__global__ void __launch_bounds__(kMaxWaves * 64) stream_kernel(StepArgs a) {
  constexpr int HS = K / 32;
  constexpr int NC = kN - K;
  constexpr int CS = UnitRaw<K, COLD>::CS;
  constexpr int CSR = CS > 0 ? CS : 1;
  constexpr bool TIERED = CS > 0;  // a cold tier with ring and flushes
  extern __shared__ float lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int hb = blockIdx.x % a.nhb, bi = blockIdx.x / a.nhb;
  const int H = a.H, P = a.P, hpw = a.hpw, c = a.c;
  const int h0 = hb * hpw, g = h0 / a.HG;
  const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
  if (slot < 0 || slot >= a.slots) {  // uniform over the workgroup
    for (int i = tid; i < hpw * P; i += blockDim.x) a.y[((size_t)bi * H + h0) * P + i] = __builtin_nanf("");
    return;
  }
  const Ws ws(a.ws, a.b, H, a.G, c);
  const int q = lane & 7, rr = lane >> 3;

  // per-lane coefficients of group g (rotated by the prep kernel)
  const float* wB = ws.B + ((size_t)bi * a.G + g) * kN;
  const float* wC = ws.C + ((size_t)bi * a.G + g) * kN;
  float Bh[HS][4], Ch[HS][4], Cc[CSR][4];
#pragma unroll
  for (int s = 0; s < HS; ++s) {
    const f4 tb = *reinterpret_cast<const f4*>(wB + 32 * s + 4 * q);
    const f4 tc = *reinterpret_cast<const f4*>(wC + 32 * s + 4 * q);
    Bh[s][0] = tb.x; Bh[s][1] = tb.y; Bh[s][2] = tb.z; Bh[s][3] = tb.w;
    Ch[s][0] = tc.x; Ch[s][1] = tc.y; Ch[s][2] = tc.z; Ch[s][3] = tc.w;
  }
#pragma unroll
  for (int s = 0; s < CSR; ++s) {
    if constexpr (CS > 0) {
      const f4 tc = *reinterpret_cast<const f4*>(wC + K + 32 * s + 4 * q);
      Cc[s][0] = tc.x; Cc[s][1] = tc.y; Cc[s][2] = tc.z; Cc[s][3] = tc.w;
    } else {
      Cc[s][0] = Cc[s][1] = Cc[s][2] = Cc[s][3] = 0.f;
    }
  }

  const float* hdb = ws.hd + ((size_t)bi * H + h0) * HD_STRIDE;
  const int RG = P >> 3;
  const int units = hpw * RG;
  bool flush = false;
  if constexpr (TIERED) {
    for (int j = 0; j < hpw; ++j) flush |= hdb[j * HD_STRIDE + HD_FLUSH] != 0.f;
  }

  if (!flush) {
    // U units per wave in flight: all their loads are issued before any compute
    constexpr int U = NSSM_UNROLL;
    for (int u0 = wave; u0 < units; u0 += U * nw) {
      UnitRaw<K, COLD> d[U];
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int u = u0 + i * nw;
        if (u < units) {
          const int j = u / RG;
          const int p = (u - j * RG) * 8 + rr;
          unit_load<K, COLD>(a, ((size_t)slot * H + h0 + j) * P + p, ((size_t)bi * H + h0 + j) * P + p, q, d[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int u = u0 + i * nw;
        if (u < units) {
          const int j = u / RG;
          const int p = (u - j * RG) * 8 + rr;
          const float* hd = hdb + j * HD_STRIDE;
          uint16_t* rx = nullptr;
          if constexpr (TIERED) rx = a.ring_x + (((size_t)slot * H + h0 + j) * c + (int)hd[HD_POS]) * P;
          unit_compute<K, COLD, false>(a, ((size_t)slot * H + h0 + j) * P + p, ((size_t)bi * H + h0 + j) * P + p,
                                       p, q, d[i], rx, hd, Bh, Ch, Cc, nullptr, nullptr, 0);
        }
      }
    }
  } else if constexpr (TIERED) {
    // the first unit's state loads go out before the window staging
    UnitRaw<K, COLD> dcur;
    if (wave < units) {
      const int j = wave / RG, p = (wave - j * RG) * 8 + rr;
      unit_load<K, COLD>(a, ((size_t)slot * H + h0 + j) * P + p, ((size_t)bi * H + h0 + j) * P + p, q, dcur);
    }
    // stage the flush window, tokens i = 0..m-1 (the last is this token):
    // rotated B cold columns of the group and w_i dt_i x_i of each head; the
    // buffered tokens sit at ring positions [c-m, c-1)
    const int m = min(max((int)hdb[HD_M], 1), c);
    float* sBc = lds;          // [m][NC]
    float* sU = lds + c * NC;  // [hpw][m][P]
    const size_t rb = ((size_t)slot * a.G + g) * c + (c - m);
    for (int i = tid; i < m * NC; i += blockDim.x) {
      const int e = i / NC, n = i - e * NC;
      sBc[i] = e < m - 1 ? a.ring_b[rb * NC + i] : wB[K + n];
    }
    for (int i = tid; i < hpw * m * P; i += blockDim.x) {
      const int j = i / (m * P), r = i - j * m * P, e = r / P, p = r - e * P;
      const uint16_t xv = e < m - 1 ? a.ring_x[(((size_t)slot * H + h0 + j) * c + (c - m + e)) * P + p]
                                    : a.x[((size_t)bi * H + h0 + j) * P + p];
      sU[i] = ws.w[((size_t)bi * H + h0 + j) * c + e] * bf2f(xv);
    }
    __syncthreads();
    // c >= 16: the window contraction Delta[p][n] = sum_i sU[i][p] sBc[i][n] runs on the
    // matrix cores (v_mfma_f32_16x16x4_f32: A = sBc^T 16 n x 4 tokens, B = sU 4 tokens
    // x 16 p, K = window tokens, zero past m). Each wave keeps up to kMfmaTiles 16 x 16
    // output tiles in registers; after a barrier they go to LDS (rows of stride
    // NC + 4, over the staging area) for the streaming-layout apply below.
    const float* dS = nullptr;
    constexpr int NT = NC / 16;
    const int ntiles = (P / 16) * NT;
    if (c >= 16 && hpw == 1 && ntiles <= nw * kMfmaTiles) {
      const int li = lane & 15, lk = lane >> 4;
      f4 acc[kMfmaTiles];
#pragma unroll
      for (int i = 0; i < kMfmaTiles; ++i) {
        acc[i] = f4{0.f, 0.f, 0.f, 0.f};
        const int tt = wave + i * nw;
        if (tt < ntiles) {
          const int pt = tt / NT, nt = tt - pt * NT;
          for (int k0 = 0; k0 < m; k0 += 4) {
            const int kk = k0 + lk;
            const int kc = kk < m ? kk : m - 1;
            float av = sBc[kc * NC + nt * 16 + li];
            float bv = sU[kc * P + pt * 16 + li];
            if (kk >= m) av = bv = 0.f;
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[i], 0, 0, 0);
          }
        }
      }
      __syncthreads();  // every wave is done reading sBc / sU
      float* dW = lds;  // [P][NC + 4]
#pragma unroll
      for (int i = 0; i < kMfmaTiles; ++i) {
        const int tt = wave + i * nw;
        if (tt < ntiles) {  // lane holds Delta[p0 + li][n0 + 4 lk .. +3]
          const int pt = tt / NT, nt = tt - pt * NT;
          *reinterpret_cast<f4*>(dW + (pt * 16 + li) * (NC + 4) + nt * 16 + 4 * lk) = acc[i];
        }
      }
      __syncthreads();
      dS = dW;
    }
    // software pipeline: the next unit's loads are in flight during this one's compute
    for (int u = wave; u < units; u += nw) {
      UnitRaw<K, COLD> dnext;
      const int un = u + nw;
      if (un < units) {
        const int j = un / RG, p = (un - j * RG) * 8 + rr;
        unit_load<K, COLD>(a, ((size_t)slot * H + h0 + j) * P + p, ((size_t)bi * H + h0 + j) * P + p, q, dnext);
      }
      const int j = u / RG;
      const int p = (u - j * RG) * 8 + rr;
      const size_t row = ((size_t)slot * H + h0 + j) * P + p;
      const size_t yrow = ((size_t)bi * H + h0 + j) * P + p;
      const float* hd = hdb + j * HD_STRIDE;
      if (hd[HD_FLUSH] != 0.f) {
        unit_compute<K, COLD, true>(a, row, yrow, p, q, dcur, nullptr, hd, Bh, Ch, Cc, sU + (size_t)j * m * P, sBc,
                                    m, dS);
      } else {
        uint16_t* rx = a.ring_x + (((size_t)slot * H + h0 + j) * c + (int)hd[HD_POS]) * P;
        unit_compute<K, COLD, false>(a, row, yrow, p, q, dcur, rx, hd, Bh, Ch, Cc, nullptr, nullptr, 0);
      }
      dcur = dnext;
    }
  }
}

// join: full state -> tiers; one workgroup per (request, head)
__global__ void join_kernel(StepArgs a, const float* __restrict__ S, const int32_t* __restrict__ phase, int K,
                            int kind) {
  const int bi = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int slot = a.slot_ids ? a.slot_ids[bi] : bi;
  if (slot < 0 || slot >= a.slots) return;
  const int NC = kN - K;
  const float* src = S + ((size_t)bi * a.H + h) * a.P * kN;
  const size_t row0 = ((size_t)slot * a.H + h) * a.P;
  // element pass (coalesced): hot columns, and the fp32 cold copy or master
  for (int i = threadIdx.x; i < a.P * kN; i += blockDim.x) {
    const int p = i / kN, n = i - p * kN;
    const float v = src[i];
    if (n < K) {
      a.hot[(row0 + p) * K + n] = v;
    } else if (kind != NSSM_COLD_NONE) {
      float* dst = kind == NSSM_COLD_FP32 ? static_cast<float*>(a.cold) : a.master;
      dst[(row0 + p) * NC + (n - K)] = v;
      if (kind == NSSM_COLD_BF16) static_cast<uint16_t*>(a.cold)[(row0 + p) * NC + (n - K)] = nssm_f32_to_bf16(v);
    }
  }
  if (kind == NSSM_COLD_FP8) {  // row pass: per-row amax scale, scale/vllm_v4_patch.py:106-111
    for (int p = threadIdx.x; p < a.P; p += blockDim.x) {
      const float* r = src + (size_t)p * kN + K;
      float am = 0.f;
      for (int n = 0; n < NC; ++n) am = fmaxf(am, fabsf(r[n]));
      const float sc = am / 448.0f + 1e-12f;
      uint8_t* d8 = static_cast<uint8_t*>(a.cold) + (row0 + p) * NC;
      for (int n = 0; n < NC; ++n) d8[n] = nssm_f32_to_e4m3fn(r[n] / sc);
      a.scale[row0 + p] = sc;
    }
  }
  if (threadIdx.x == 0) {
    const size_t o = (size_t)slot * a.H + h;
    a.t[o] = phase ? phase[bi] : 0;
    a.nv[o] = 0;
    a.glog[o] = 0.f;
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
  const int nv = min(max(a.nv[o], 0), c - 1);
  const int t0 = max(a.t[o] - nv, 0);  // step count at the snapshot; pending token i sits at ring (t0 + i) % c
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
    const float* cm = kind == NSSM_COLD_FP32 ? static_cast<const float*>(a.cold) + row * NC : a.master + row * NC;
    for (int n = 0; n < NC; ++n) {
      float v = dtot * cm[n];
      for (int i = 0; i < nv; ++i) {
        const int pos = (t0 + i) % c;
        const float u = w[i] * bf2f(a.ring_x[(rh + pos) * a.P + p]);
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
// host side
int g_hpw_override = 0, g_waves_override = 0;
constexpr size_t kMaxLds = 64 * 1024;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_params(const nssm_layer_params* prm) {
  if (!prm || !prm->dt_bias || !prm->A || !prm->D) return NSSM_E_NULL;
  if (prm->N != kN || prm->H <= 0 || prm->G <= 0 || prm->H % prm->G || prm->H / prm->G > 64) return NSSM_E_DIMS;
  if (prm->P <= 0 || prm->P % 16 || prm->P > 256) return NSSM_E_DIMS;
  if (prm->R && !aligned16(prm->R)) return NSSM_E_ALIGN;
  return NSSM_OK;
}

int check_inputs(const nssm_step_inputs* in, const float* y) {
  if (!in || !in->x || !in->B || !in->C || !in->dt || !y) return NSSM_E_NULL;
  if (in->b < 0) return NSSM_E_DIMS;
  return NSSM_OK;
}

int check_ws(const nssm_layer_params* prm, int b, int c, const void* ws, int64_t ws_bytes) {
  if (!ws) return NSSM_E_WORKSPACE;
  if (!aligned16(ws)) return NSSM_E_ALIGN;
  if (ws_bytes < (int64_t)(ws_floats(b, prm->H, prm->G, c) * sizeof(float))) return NSSM_E_WORKSPACE;
  return NSSM_OK;
}

// largest divisor of n not above cap
int divisor_at_most(int n, int cap) {
  for (int d = cap < n ? cap : n; d >= 1; --d)
    if (n % d == 0) return d;
  return 1;
}

size_t stream_lds_bytes(int hpw, int P, int c, int K, int kind = NSSM_COLD_FP32) {
  const int NC = kN - K;
  if (NC <= 0 || kind == NSSM_COLD_NONE) return 0;
  size_t fl = (size_t)c * NC + (size_t)hpw * c * P;  // window staging
  if (c >= 16 && hpw == 1) fl = fl > (size_t)P * (NC + 4) ? fl : (size_t)P * (NC + 4);  // MFMA exchange
  return fl * sizeof(float);
}

struct Launch {
  int hpw, waves;
};

int pick_launch(int H, int G, int P, int K, int c, Launch* out, int kind = NSSM_COLD_FP32) {
  const int HG = H / G, RG = P / 8;
  int hpw = 1;
  if (g_hpw_override > 0) {
    if (HG % g_hpw_override) return NSSM_E_TUNING;
    hpw = g_hpw_override;
  }
  while (hpw > 1 && stream_lds_bytes(hpw, P, c, K, kind) > kMaxLds) hpw = divisor_at_most(HG, hpw - 1);
  if (stream_lds_bytes(hpw, P, c, K, kind) > kMaxLds) return NSSM_E_DIMS;
  // measured on MI355X at the 9B shape (P = 80): the untiered stream runs best
  // with two units per wave (5 waves per head), the tiered one with 4 waves
  const int waves = g_waves_override > 0 ? g_waves_override
                    : K < kN && kind != NSSM_COLD_NONE ? (hpw * RG < 4 ? hpw * RG : 4)
                                         : divisor_at_most(hpw * RG, 5);
  if (waves > kMaxWaves) return NSSM_E_TUNING;
  out->hpw = hpw;
  out->waves = waves;
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
  if (tr->cold_kind < NSSM_COLD_FP32 || tr->cold_kind > NSSM_COLD_NONE) return NSSM_E_KIND;
  const bool cold = tr->cold_kind != NSSM_COLD_NONE;
  if (!tr->hot || !tr->t || !tr->nv || !tr->glog || (cold && !tr->cold)) return NSSM_E_NULL;
  if (cold && need_ring && (!tr->ring_x || !tr->ring_dt || !tr->ring_b)) return NSSM_E_NULL;
  if ((tr->cold_kind == NSSM_COLD_BF16 || tr->cold_kind == NSSM_COLD_FP8) && !tr->master) return NSSM_E_NULL;
  if (tr->cold_kind == NSSM_COLD_FP8 && !tr->scale) return NSSM_E_NULL;
  if (tr->slots <= 0 || tr->c < 1 || tr->c > kMaxC) return NSSM_E_DIMS;
  if (tr->k_hot != 32 && tr->k_hot != 64 && tr->k_hot != 96) return NSSM_E_DIMS;
  if (!aligned16(tr->hot) || (cold && !aligned16(tr->cold)) || (tr->master && !aligned16(tr->master)))
    return NSSM_E_ALIGN;
  return NSSM_OK;
}

void fill_tier(StepArgs& a, const nssm_tier* tr) {
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
}

template <int K, int COLD>
int launch_pair(const StepArgs& a, int waves, hipStream_t st) {
  constexpr bool TIERED = K < kN && COLD != NSSM_COLD_NONE;
  if (a.b == 0) return NSSM_OK;
  hipLaunchKernelGGL((prep_kernel<TIERED>), dim3((unsigned)a.b * a.G), dim3(kPrepThreads), 0, st, a);
  hipLaunchKernelGGL((stream_kernel<K, COLD>), dim3((unsigned)a.b * a.nhb), dim3(waves * 64),
                     stream_lds_bytes(a.hpw, a.P, a.c, K, COLD), st, a);
  return hipGetLastError() == hipSuccess ? NSSM_OK : NSSM_E_LAUNCH;
}

template <int K>
int dispatch_kind(const StepArgs& a, int kind, int waves, hipStream_t st) {
  switch (kind) {
    case NSSM_COLD_FP32: return launch_pair<K, NSSM_COLD_FP32>(a, waves, st);
    case NSSM_COLD_BF16: return launch_pair<K, NSSM_COLD_BF16>(a, waves, st);
    case NSSM_COLD_FP8: return launch_pair<K, NSSM_COLD_FP8>(a, waves, st);
    case NSSM_COLD_NONE: return launch_pair<K, NSSM_COLD_NONE>(a, waves, st);
  }
  return NSSM_E_KIND;
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
    case NSSM_E_ALIGN: return "a state, parameter or workspace pointer is not 16-byte aligned";
    case NSSM_E_KIND: return "unknown cold storage kind";
    case NSSM_E_LAUNCH: return "HIP kernel launch failed";
    case NSSM_E_TUNING: return "launch override does not fit the dimensions";
    case NSSM_E_WORKSPACE: return "workspace missing or smaller than nssm_step_workspace_bytes()";
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
  if (slots <= 0 || H <= 0 || P <= 0 || N != kN || G <= 0 || k_hot <= 0 || k_hot >= N || c < 1 || c > kMaxC)
    return NSSM_E_DIMS;
  if (cold_kind < NSSM_COLD_FP32 || cold_kind > NSSM_COLD_NONE) return NSSM_E_KIND;
  const int64_t rows = (int64_t)slots * H * P;
  const int64_t NC = N - k_hot;
  const int64_t esz = cold_kind == NSSM_COLD_FP32 ? 4 : cold_kind == NSSM_COLD_BF16 ? 2 : cold_kind == NSSM_COLD_FP8 ? 1 : 0;
  const int64_t ring = cold_kind == NSSM_COLD_NONE ? 0 : 1;
  sz[0] = rows * k_hot * 4;
  sz[1] = rows * NC * esz;
  sz[2] = cold_kind == NSSM_COLD_FP8 ? rows * 4 : 0;
  sz[3] = cold_kind == NSSM_COLD_BF16 || cold_kind == NSSM_COLD_FP8 ? rows * NC * 4 : 0;
  sz[4] = ring * slots * H * c * P * 2;
  sz[5] = ring * slots * H * c * 4;
  sz[6] = ring * slots * G * c * NC * 4;
  sz[7] = (int64_t)slots * H * 4;
  sz[8] = (int64_t)slots * H * 4;
  sz[9] = (int64_t)slots * H * 4;
  return NSSM_OK;
}

int nssm_set_launch(int32_t heads_per_wg, int32_t waves_per_wg) {
  if (heads_per_wg < 0 || waves_per_wg < 0 || waves_per_wg > kMaxWaves) return NSSM_E_TUNING;
  g_hpw_override = heads_per_wg;
  g_waves_override = waves_per_wg;
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
  if ((rc = pick_launch(prm->H, prm->G, prm->P, kN, 0, &L))) return rc;
  a.hpw = L.hpw;
  a.nhb = prm->H / L.hpw;
  return launch_pair<kN, NSSM_COLD_FP32>(a, L.waves, (hipStream_t)stream);
}

int nssm_v4_step(const nssm_layer_params* prm, const nssm_tier* tier, const nssm_step_inputs* in, float* y,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_params(prm);
  if (rc) return rc;
  if ((rc = check_inputs(in, y))) return rc;
  if ((rc = check_tier(tier, true))) return rc;
  if (!in->slot_ids && in->b > tier->slots) return NSSM_E_DIMS;
  if ((rc = check_ws(prm, in->b, tier->c, workspace, workspace_bytes))) return rc;
  StepArgs a = {};
  fill_common(a, prm, in, y, workspace);
  fill_tier(a, tier);
  Launch L;
  if ((rc = pick_launch(prm->H, prm->G, prm->P, tier->k_hot, tier->c, &L, tier->cold_kind))) return rc;
  a.hpw = L.hpw;
  a.nhb = prm->H / L.hpw;
  hipStream_t st = (hipStream_t)stream;
  switch (tier->k_hot) {
    case 32: return dispatch_kind<32>(a, tier->cold_kind, L.waves, st);
    case 64: return dispatch_kind<64>(a, tier->cold_kind, L.waves, st);
    case 96: return dispatch_kind<96>(a, tier->cold_kind, L.waves, st);
  }
  return NSSM_E_DIMS;
}

int nssm_v4_join(const nssm_layer_params* prm, const nssm_tier* tier, const float* state, int32_t b,
                 const int32_t* slot_ids, const int32_t* phase, void* stream) {
  int rc = check_params(prm);
  if (rc) return rc;
  if ((rc = check_tier(tier, false))) return rc;
  if (!state) return NSSM_E_NULL;
  if (b < 0 || (!slot_ids && b > tier->slots)) return NSSM_E_DIMS;
  if (b == 0) return NSSM_OK;
  StepArgs a = {};
  fill_tier(a, tier);
  a.slot_ids = slot_ids;
  a.H = prm->H;
  a.P = prm->P;
  a.G = prm->G;
  a.HG = prm->H / prm->G;
  hipLaunchKernelGGL(join_kernel, dim3((unsigned)b * prm->H), dim3(128), 0, (hipStream_t)stream, a, state, phase,
                     (int)tier->k_hot, (int)tier->cold_kind);
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
  fill_tier(a, tier);
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

int nssm_rotate(const uint16_t* in, const float* R, float* out, int32_t T, int32_t G, int32_t N, void* stream) {
  if (!in || !R || !out) return NSSM_E_NULL;
  if (T < 0 || G <= 0 || N <= 0 || N > 1024) return NSSM_E_DIMS;
  if (T == 0) return NSSM_OK;
  hipLaunchKernelGGL(rotate_kernel, dim3((unsigned)T * G), dim3(128), N * sizeof(float), (hipStream_t)stream, in,
                     R, out, G, N);
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
