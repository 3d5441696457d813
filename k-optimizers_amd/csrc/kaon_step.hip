// kaon_step.hip -- gfx950 kernels of the fused optimizer step (Adakaon,
// Nekaon's fused lookahead, Lion) and the C-ABI entry points that launch them.
//
// Reference (K-Optimizers "kaon" 0.7.4) semantics followed, per element:
//   Adakaon  src/kaon/adakaon.py:968-1014 (batched twin :840-966)
//   Lion     src/kaon/lion.py:454-485 (batched twin :416-451)
//   Nekaon   src/kaon/msam.py:202-235, 375-406; src/kaon/nekaon.py:162-171
//   codecs   src/kaon/_momentum_codec.py:72-200, 253-406
//   writes   src/kaon/_backend.py:82-142, _stochastic_rounding.py:70-103
//   factored src/kaon/_factored.py:26-83; GC src/kaon/_backend.py:147-177
//
// One step of one param group runs as a short sequence of multi-tensor
// launches, each covering every tensor of the group through a work-item table
// (the descriptor table replaces the reference's per-role pointer arrays):
//   phase 1  row items   GC row means, row second-moment EMA, column partials
//   phase 2  fin items   column EMA + column factors; row-mean + row factors
//   phase 3  row items   per-row sum of U^2 (U = G*r*c) for the RMS clip
//   phase 4  per tensor  clip divisor
//   phase 5  flat items  cautious keep-count, momentum absmax, old-scale copy
//   phase 6  flat items  requant + momentum write, cautious rescale, weight
//                        write (SR / RN / kahan / fp32), Nekaon remove+climb
// Reductions follow one fixed order (the canonical order of the CPU oracle);
// there are no floating-point atomics, so results are deterministic.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>

#include "kaon_device.h"

using namespace kaon;

thread_local std::string g_err;

// Error text shared with the planner (kaon_plan.cpp).
void kaon_set_error(const std::string& s) { g_err = s; }

namespace {

int fail(const char* what, hipError_t e = hipSuccess) {
  g_err = what;
  if (e != hipSuccess) {
    g_err += ": ";
    g_err += hipGetErrorString(e);
  }
  return e != hipSuccess ? (int)e : -1;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(what, e);
  return 0;
}

// ------------------------------------------------------------ workspace views
struct Ws {
  float* base;
  __device__ float* mu(const KaonTensor& T) const { return base + T.ws_row; }
  __device__ float* rf(const KaonTensor& T) const { return base + T.ws_row + T.R; }
  __device__ float* rs(const KaonTensor& T) const { return base + T.ws_row + 2 * T.R; }
  __device__ uint32_t* ramax(const KaonTensor& T) const { return (uint32_t*)(base + T.ws_row + 3 * T.R); }
  __device__ float* roldsc(const KaonTensor& T) const { return base + T.ws_row + 4 * T.R; }
  __device__ float* cf(const KaonTensor& T) const { return base + T.ws_col; }
  __device__ float* part(const KaonTensor& T) const { return base + T.ws_part; }
  __device__ uint32_t* bamax(const KaonTensor& T) const { return (uint32_t*)(base + T.ws_blk); }
  __device__ float* boldsc(const KaonTensor& T, int64_t nb) const { return base + T.ws_blk + nb; }
  __device__ float* scal(const KaonTensor& T) const { return base + T.ws_scal; }
};

template <int DT>
__device__ __forceinline__ float round_to(float x) {
  return DT == KAON_BF16 ? rbf(x) : x;
}

__device__ __forceinline__ int64_t nblocks4(const KaonTensor& T) {
  return (T.n + T.block4 - 1) / T.block4;
}

// Zero what later phases accumulate with atomics (keep-count, absmax).  Run by
// the phase-1 item that owns rows [row0, row0+nrows).
__device__ void zero_accumulators(const KaonTensor& T, const KaonItem& it, const Ws& ws, int codec) {
  if (it.row0 == 0 && threadIdx.x == 0) ((uint32_t*)ws.scal(T))[1] = 0u;
  if (codec == KAON_MOM_INT8) {
    for (int i = threadIdx.x; i < it.nrows; i += KAON_WG) ws.ramax(T)[it.row0 + i] = 0u;
  } else if (codec == KAON_MOM_4BIT) {
    const int64_t e_begin = (int64_t)it.row0 * T.C;
    const int64_t e_end = (int64_t)(it.row0 + it.nrows) * T.C;
    const int64_t b0 = e_begin / T.block4, b1 = (e_end - 1) / T.block4;
    for (int64_t b = b0 + threadIdx.x; b <= b1; b += KAON_WG) ws.bamax(T)[b] = 0u;
  }
}

// =============================================================== phase 1
// Row items.  mode 0 (Adakaon): GC row mean (stored), row EMA of mean_C(G^2),
// column partial sums of KAON_COLGROUP rows; 1-D tensors: v EMA.  mode 1
// (Lion): GC row mean only.  KM bounds the chunks per thread kept in
// registers (C <= 2048*KM).
template <int GT, int KM>
__global__ __launch_bounds__(KAON_WG) void k_rows(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws,
                                                  KaonHyper hp, int mode) {
  __shared__ float lds4[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  zero_accumulators(T, it, ws, hp.codec);
  const int64_t C = T.C;
  const bool eps = (hp.flags & KAON_F_EPS) != 0;

  if (!T.factored) {
    const bool vec = T.vec_flat != 0;
    if (mode != 0) return;
    // v = lerp(v, g*g (+eps1), 1-beta2)  (adakaon.py:990-995)
    const int64_t nch = (C + 7) >> 3;
    for (int64_t c = threadIdx.x; c < nch; c += KAON_WG) {
      const int64_t j0 = c * 8;
      const int cnt = (int)min<int64_t>(8, C - j0);
      const bool vv = vec && cnt == 8;
      float x[8], v[8];
      ld8<GT>(T.g, j0, cnt, vv, x);
      ld8<KAON_F32>(T.v, j0, cnt, vv, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float q = x[i] * x[i];
        if (eps) q = q + hp.eps1;
        v[i] = klerp(v[i], q, hp.w2);
      }
      st8_f32(T.v, j0, cnt, vv, v);
    }
    return;
  }

  const bool gc = (hp.flags & KAON_F_GC) != 0;
  if (mode == 1 && !gc) return;
  const bool vec = T.vec_rows != 0;
  const int64_t nch = (C + 7) >> 3;
  float* mu_arr = ws.mu(T);
  float colacc[KM][8];
#pragma unroll
  for (int k = 0; k < KM; ++k)
#pragma unroll
    for (int i = 0; i < 8; ++i) colacc[k][i] = 0.0f;

  for (int rr = 0; rr < it.nrows; ++rr) {
    const int64_t r = (int64_t)it.row0 + rr;
    const int64_t rowoff = r * C;
    float x[KM][8];
    int cntk[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      const int64_t c = threadIdx.x + (int64_t)KAON_WG * k;
      const int64_t j0 = c * 8;
      const int cnt = c < nch ? (int)min<int64_t>(8, C - j0) : 0;
      cntk[k] = cnt;
      if (cnt > 0) {
        ld8<GT>(T.g, rowoff + j0, cnt, vec && cnt == 8, x[k]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[k][i] = 0.0f;
      }
    }
    if (gc) {
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < KM; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i < cntk[k]) a = a + x[k][i];
      const float s = csum_finish(a, nch, lds4);
      const float mu = round_to<GT>(s / (float)C);
      if (threadIdx.x == 0) mu_arr[r] = mu;
#pragma unroll
      for (int k = 0; k < KM; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i < cntk[k]) x[k][i] = round_to<GT>(x[k][i] - mu);
    }
    if (mode == 1) continue;
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < cntk[k]) {
          float q = x[k][i] * x[k][i];
          if (eps) q = q + hp.eps1;
          x[k][i] = q;
          a = a + q;
        }
    const float s2 = csum_finish(a, nch, lds4);
    if (threadIdx.x == 0) T.row[r] = klerp(T.row[r], s2 / (float)C, hp.w2);
#pragma unroll
    for (int k = 0; k < KM; ++k)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < cntk[k]) colacc[k][i] = colacc[k][i] + x[k][i];
  }
  if (mode == 1) return;
  float* part = ws.part(T) + (int64_t)(it.row0 / KAON_COLGROUP) * C;
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const int64_t c = threadIdx.x + (int64_t)KAON_WG * k;
    if (c >= nch) continue;
    const int64_t j0 = c * 8;
    const int cnt = (int)min<int64_t>(8, C - j0);
    st8_f32(part, j0, cnt, vec && cnt == 8, colacc[k]);
  }
}

// =============================================================== phase 2
// Finalize items.  kind 0: col = lerp(col, colsum/R, 1-beta2), cf = 1/sqrt(col)
// for columns [row0, row0+nrows).  kind 1: rm = mean(row) (canonical sum),
// rf = 1/sqrt(row/rm) (_factored.py:48-52, 76-82).
__global__ __launch_bounds__(KAON_WG) void k_fin(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ float lds4[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t R = T.R, C = T.C;
  if (it.kind == 0) {
    const float* part = ws.part(T);
    float* cf = ws.cf(T);
    for (int64_t j = it.row0 + threadIdx.x; j < (int64_t)it.row0 + it.nrows; j += KAON_WG) {
      float cs = 0.0f;
      for (int g = 0; g < T.ngroups; ++g) cs = cs + part[(int64_t)g * C + j];
      const float nc = klerp(T.col[j], cs / (float)R, hp.w2);
      T.col[j] = nc;
      cf[j] = 1.0f / sqrtf(nc);
    }
  } else {
    const int64_t nch = (R + 7) >> 3;
    float a = 0.0f;
    for (int64_t c = threadIdx.x; c < nch; c += KAON_WG)
      for (int i = 0; i < 8; ++i) {
        const int64_t j = c * 8 + i;
        if (j < R) a = a + T.row[j];
      }
    const float rm = csum_finish(a, nch, lds4) / (float)R;
    float* rf = ws.rf(T);
    for (int64_t i = threadIdx.x; i < R; i += KAON_WG) rf[i] = 1.0f / sqrtf(T.row[i] / rm);
  }
}

// =============================================================== phase 3
// Row items: rs[r] = canonical sum over the row of U^2, U = (G*rf)*cf
// (factored) or G*(1/sqrt(v)) (1-D; the whole tensor is one row).
template <int GT>
__global__ __launch_bounds__(KAON_WG) void k_ss(const KaonTensor* __restrict__ D,
                                                const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ float lds4[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C;
  const bool vec = T.factored ? T.vec_rows != 0 : T.vec_flat != 0;
  const bool gc = (hp.flags & KAON_F_GC) && T.factored;
  const int64_t nch = (C + 7) >> 3;
  const float* cfa = ws.cf(T);
  for (int rr = 0; rr < it.nrows; ++rr) {
    const int64_t r = (int64_t)it.row0 + rr;
    const float mu = gc ? ws.mu(T)[r] : 0.0f;
    const float rf = T.factored ? ws.rf(T)[r] : 0.0f;
    float a = 0.0f;
    for (int64_t c = threadIdx.x; c < nch; c += KAON_WG) {
      const int64_t j0 = c * 8;
      const int cnt = (int)min<int64_t>(8, C - j0);
      const bool vv = vec && cnt == 8;
      float x[8], f[8];
      ld8<GT>(T.g, r * C + j0, cnt, vv, x);
      if (T.factored) ld8<KAON_F32>(cfa, j0, cnt, vv, f);
      else ld8<KAON_F32>(T.v, j0, cnt, vv, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i >= cnt) break;
        float g = x[i];
        if (gc) g = round_to<GT>(g - mu);
        const float u = T.factored ? (g * rf) * f[i] : g * (1.0f / sqrtf(f[i]));
        a = a + u * u;
      }
    }
    const float s = csum_finish(a, nch, lds4);
    if (threadIdx.x == 0) ws.rs(T)[r] = s;
  }
}

// =============================================================== phase 4
// One workgroup per tensor: fac = max(sqrt(sum_r rs[r]) / sqrt(n) / clip, 1)
// (_backend.py:45-47; adakaon.py:1000-1002).
__global__ __launch_bounds__(KAON_WG) void k_fac(const KaonTensor* __restrict__ D, Ws ws, KaonHyper hp) {
  __shared__ float lds4[4];
  const KaonTensor& T = D[blockIdx.x];
  const int64_t R = T.R;
  const float* rs = ws.rs(T);
  const int64_t nch = (R + 7) >> 3;
  float a = 0.0f;
  for (int64_t c = threadIdx.x; c < nch; c += KAON_WG)
    for (int i = 0; i < 8; ++i) {
      const int64_t j = c * 8 + i;
      if (j < R) a = a + rs[j];
    }
  const float ss = csum_finish(a, nch, lds4);
  if (threadIdx.x == 0) {
    const float rmsv = sqrtf(ss) / T.sqrt_n;
    ws.scal(T)[0] = fmaxf(rmsv / hp.clip, 1.0f);
  }
}

// =============================================================== phases 5/6
// Per-chunk row/block context resolved once when a chunk lies in one row.
struct RowCtx {
  float mu, rf;     // GC mean, row factor
  float oldsc;      // int8 scale before this step (per row)
  float newsc;      // int8 scale after requant
  double rnew;      // RN64(1/newsc)
};

// Momentum chunk load: fp32 values of the OLD momentum given per-element
// scales (int8: per-row, 4-bit: per-block).
template <int CODEC>
__device__ __forceinline__ void ld_mom_raw(const KaonTensor& T, int64_t e0, int cnt, bool vec, uint32_t q[8]) {
  if (CODEC == KAON_MOM_INT8) {
    const int8_t* m = (const int8_t*)T.m + e0;
    if (vec) {
      const uint2 v = *(const uint2*)m;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q[i] = (v.x >> (8 * i)) & 0xFFu;
        q[4 + i] = (v.y >> (8 * i)) & 0xFFu;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = i < cnt ? (uint32_t)(uint8_t)m[i] : 0u;
    }
  } else if (CODEC == KAON_MOM_4BIT) {
    const uint8_t* m = (const uint8_t*)T.m + (e0 >> 1);
    if (vec) {
      const uint32_t v = *(const uint32_t*)m;
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = (v >> (4 * i)) & 0xFu;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = i < cnt ? ((uint32_t)m[i >> 1] >> (4 * (i & 1))) & 0xFu : 8u;
    }
  } else if (CODEC == KAON_MOM_BF16) {
    ld8_bits(T.m, e0, cnt, vec, q);
  } else if (CODEC == KAON_MOM_F32) {
    float f[8];
    ld8<KAON_F32>(T.m, e0, cnt, vec, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = __float_as_uint(f[i]);
  }
}

template <int CODEC>
__device__ __forceinline__ void st_mom_raw(const KaonTensor& T, int64_t e0, int cnt, bool vec, const uint32_t q[8]) {
  if (CODEC == KAON_MOM_INT8) {
    int8_t* m = (int8_t*)T.m + e0;
    if (vec) {
      uint2 v;
      v.x = (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | ((q[3] & 0xFF) << 24);
      v.y = (q[4] & 0xFF) | ((q[5] & 0xFF) << 8) | ((q[6] & 0xFF) << 16) | ((q[7] & 0xFF) << 24);
      *(uint2*)m = v;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < cnt) m[i] = (int8_t)q[i];
    }
  } else if (CODEC == KAON_MOM_4BIT) {
    uint8_t* m = (uint8_t*)T.m + (e0 >> 1);
    if (vec) {
      uint32_t v = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) v |= (q[i] & 0xFu) << (4 * i);
      *(uint32_t*)m = v;
    } else {
      // the chunk owns bytes e0/2 .. (e0+cnt-1)/2 (e0 even); a dangling high
      // nibble of an odd-length tensor is written as 0 (_pack_nibbles pads 0)
      for (int b = 0; 2 * b < cnt; ++b) {
        const uint32_t lo = q[2 * b] & 0xFu;
        const uint32_t hi = (2 * b + 1 < cnt) ? (q[2 * b + 1] & 0xFu) : 0u;
        m[b] = (uint8_t)(lo | (hi << 4));
      }
    }
  } else if (CODEC == KAON_MOM_BF16) {
    st8_bits(T.m, e0, cnt, vec, q);
  } else if (CODEC == KAON_MOM_F32) {
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(q[i]);
    st8_f32(T.m, e0, cnt, vec, f);
  }
}

// MSAM perturbation value: clamp(nan_to_num(x, 0, +b, -b), -b, b) (msam.py:222-230).
__device__ __forceinline__ float msam_e(float x, float bound) {
  if (x != x) return 0.0f;
  if (isinf(x)) return x > 0.0f ? bound : -bound;
  return fminf(fmaxf(x, -bound), bound);
}

// Flat items over [row0, row0 + nrows) elements of one tensor (row0/nrows hold
// the flat start and length).  OPT: KAON_OPT_ADAKAON (also Nekaon) or
// KAON_OPT_LION.  PHASE 5: keep-count + absmax + old-scale copy.  PHASE 6:
// write momentum and weights.
#define KAON_LDS_AMAX 2048

template <int OPT, int PHASE, int PT, int GT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_flat(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ uint32_t lds_amax[KAON_LDS_AMAX];
  __shared__ uint32_t lds4[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C, n = T.n;
  const int64_t e_begin = it.row0, e_end = (int64_t)it.row0 + it.nrows;
  const bool vecT = T.vec_flat != 0;
  const bool factored = T.factored != 0;
  const bool gc = (hp.flags & KAON_F_GC) && factored;
  const bool cautious = (hp.flags & KAON_F_CAUTIOUS) != 0;
  const bool wd = (hp.flags & KAON_F_WD) != 0;
  const bool mom = (hp.flags & KAON_F_MOMENTUM) != 0 && CODEC != KAON_MOM_NONE;
  const bool nk_remove = OPT == KAON_OPT_ADAKAON && mom && (hp.flags & KAON_F_NK_REMOVE);
  const bool nk_climb = OPT == KAON_OPT_ADAKAON && mom && (hp.flags & KAON_F_NK_CLIMB);
  const bool quant = mom && (CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT);
  const int64_t B = CODEC == KAON_MOM_4BIT ? (int64_t)T.block4 : 1;
  const int64_t nb = CODEC == KAON_MOM_4BIT ? nblocks4(T) : 0;

  // per-tensor scalars
  float fac = 1.0f;
  double rfac = 1.0;
  if (OPT == KAON_OPT_ADAKAON) {
    fac = ws.scal(T)[0];
    rfac = rcp64(fac);
  }
  double rden = 1.0;
  if (PHASE == 6 && cautious) {
    const uint32_t cnt = ((const uint32_t*)ws.scal(T))[1];
    const float den = fmaxf((float)cnt / (float)n, 1e-8f);
    rden = rcp64(den);
  }

  // absmax bookkeeping (phase 5, quantized codecs): entries are rows (int8) or
  // blocks (4-bit) touched by this item
  int64_t a_first = 0, a_last = -1;
  bool use_lds = false;
  if (PHASE == 5 && quant) {
    if (CODEC == KAON_MOM_INT8) {
      a_first = factored ? e_begin / C : 0;
      a_last = factored ? (e_end - 1) / C : 0;
    } else {
      a_first = e_begin / B;
      a_last = (e_end - 1) / B;
    }
    use_lds = (a_last - a_first + 1) <= KAON_LDS_AMAX;
    if (use_lds)
      for (int i = threadIdx.x; i < a_last - a_first + 1; i += KAON_WG) lds_amax[i] = 0u;
    __syncthreads();
  }
  uint32_t keep = 0;

  for (int64_t e0 = e_begin + 8 * (int64_t)threadIdx.x; e0 < e_end; e0 += 8 * KAON_WG) {
    const int cnt = (int)min<int64_t>(8, e_end - e0);
    const bool vec = vecT && cnt == 8;
    // row / column of the chunk start
    int64_t r0 = 0, j0 = e0;
    if (factored) {
      if (n < 0xFFFFFFFFll) {
        r0 = (int64_t)((uint32_t)e0 / (uint32_t)C);
      } else {
        r0 = e0 / C;
      }
      j0 = e0 - r0 * C;
    }
    const bool one_row = !factored || (j0 + cnt <= C);

    float g[8], p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    ld8<GT>(T.g, e0, cnt, vec, g);
    const bool need_p = PHASE == 6 || wd;
    uint32_t pbits[8];
    if (need_p) {
      if (PT == KAON_BF16) {
        ld8_bits(T.p, e0, cnt, vec, pbits);
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = bf2f(pbits[i]);
      } else {
        ld8<KAON_F32>(T.p, e0, cnt, vec, p);
      }
    }
    uint32_t mq[8];
    if (mom) ld_mom_raw<CODEC>(T, e0, cnt, vec, mq);
    float cf8[8];
    if (OPT == KAON_OPT_ADAKAON) {
      if (factored) {
        if (one_row && vec && (j0 & 7) == 0) {
          ld8<KAON_F32>(ws.cf(T), j0, 8, true, cf8);
        } else {
          int64_t jj = j0;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            cf8[i] = i < cnt ? ws.cf(T)[jj] : 0.0f;
            if (++jj == C) jj = 0;
          }
        }
      } else {
        ld8<KAON_F32>(T.v, e0, cnt, vec, cf8);  // holds v for 1-D
      }
    }
    // noise words (phase 6, bf16 weights)
    uint32_t nz0[8], nz1[8], nz2[8];
    const bool lowp = PT == KAON_BF16;
    if (lowp && nk_remove && need_p)
      noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 0u, e0, T.noise[0], cnt, nz0);
    if (PHASE == 6 && lowp) {
      if (hp.bf16_method == KAON_SR)
        noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 1u, e0, T.noise[1], cnt, nz1);
      if (nk_climb) noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 2u, e0, T.noise[2], cnt, nz2);
    }

    // row context
    RowCtx rc{0.0f, 0.0f, 1.0f, 1.0f, 1.0};
    int64_t rcur = -1;
    int64_t ri = r0, ji = j0;
    uint32_t qout[8];
    float dout[8];
    float mnew[8];
    float amax_chunk = 0.0f;
    int64_t amax_idx = -1;  // entry (row/block) the chunk's running max belongs to

#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i >= cnt) {
        qout[i] = mq[i];
        dout[i] = 0.0f;
        mnew[i] = 0.0f;
        continue;
      }
      const int64_t e = e0 + i;
      if (factored && ri != rcur) {
        rcur = ri;
        rc.mu = gc ? ws.mu(T)[ri] : 0.0f;
        if (OPT == KAON_OPT_ADAKAON) rc.rf = ws.rf(T)[ri];
        if (CODEC == KAON_MOM_INT8 && mom) {
          rc.oldsc = PHASE == 5 ? T.m_scale[ri] : ws.roldsc(T)[ri];
          if (PHASE == 6) {
            const float am = __uint_as_float(ws.ramax(T)[ri]);
            rc.newsc = fmaxf(am, 1e-12f) / 127.0f;
            rc.rnew = rcp64(rc.newsc);
          }
        }
      } else if (!factored && rcur < 0) {
        rcur = 0;
        if (CODEC == KAON_MOM_INT8 && mom) {
          rc.oldsc = PHASE == 5 ? T.m_scale[0] : ws.roldsc(T)[0];
          if (PHASE == 6) {
            const float am = __uint_as_float(ws.ramax(T)[0]);
            rc.newsc = fmaxf(am, 1e-12f) / 127.0f;
            rc.rnew = rcp64(rc.newsc);
          }
        }
      }
      // 4-bit block scale context (per element; blocks need not align to chunks)
      float b_oldsc = 1.0f, b_newsc = 1.0f;
      double b_rnew = 1.0;
      int64_t blk = 0;
      if (CODEC == KAON_MOM_4BIT && mom) {
        blk = e / B;
        b_oldsc = PHASE == 5 ? T.m_scale[blk] : ws.boldsc(T, nb)[blk];
        if (PHASE == 6) {
          const float am = __uint_as_float(ws.bamax(T)[blk]);
          b_newsc = fmaxf(am, 1e-12f) / 7.0f;
          b_rnew = rcp64(b_newsc);
        }
      }

      // gradient as the step sees it (GC in the grad dtype)
      float gv = g[i];
      if (gc) gv = round_to<GT>(gv - rc.mu);

      float d;       // delta (pre-cautious)
      float mfv = 0; // new momentum value (fp32, pre-requant)
      float mold = 0.0f;
      if (mom) {
        if (CODEC == KAON_MOM_INT8) mold = (float)(int8_t)(uint8_t)mq[i] * rc.oldsc;
        else if (CODEC == KAON_MOM_4BIT) mold = ((float)mq[i] - 8.0f) * b_oldsc;
        else if (CODEC == KAON_MOM_BF16) mold = bf2f(mq[i]);
        else if (CODEC == KAON_MOM_F32) mold = __uint_as_float(mq[i]);
      }
      float pw = p[i];  // weight the inner step sees (after Nekaon removal)
      if (nk_remove && need_p) {
        const float ev = msam_e(mold * hp.nk_k, hp.nk_bound_old);
        if (lowp) pw = bf2f(sr_bf16(p[i] + ev, nz0[i]));
        else pw = p[i] + ev;
      }

      if (OPT == KAON_OPT_ADAKAON) {
        const float u = factored ? (gv * rc.rf) * cf8[i] : gv * (1.0f / sqrtf(cf8[i]));
        const float ud = (fac == 1.0f ? u : div_r64(u, rfac)) * hp.lr;
        if (mom) {
          if (CODEC == KAON_MOM_BF16) {
            const uint32_t mb = f2bf(klerp(mold, rbf(ud), hp.w1));
            qout[i] = mb;
            d = bf2f(mb);
          } else {
            mfv = klerp(mold, ud, hp.w1);
            d = mfv;
            if (CODEC == KAON_MOM_F32) qout[i] = __float_as_uint(mfv);
          }
        } else {
          d = ud;
        }
        if (wd) d = __fmaf_rn(hp.wdl, pw, d);
      } else {  // Lion
        const float cdir = __fmaf_rn(hp.a1, gv, mold * hp.b1);
        d = ksign(cdir);
        mfv = __fmaf_rn(hp.a2, gv, mold * hp.b2);
        if (CODEC == KAON_MOM_F32) qout[i] = __float_as_uint(mfv);
        else if (CODEC == KAON_MOM_BF16) qout[i] = f2bf(mfv);
        if (wd) d = __fmaf_rn(hp.wdl, pw, d);
      }
      const bool kp = d * gv > 0.0f;

      if (PHASE == 5) {
        keep += kp ? 1u : 0u;
        if (quant) {
          const int64_t idx = CODEC == KAON_MOM_INT8 ? (factored ? ri : 0) : blk;
          const float ax = fabsf(mfv);
          if (idx != amax_idx) {
            if (amax_idx >= 0) {
              if (use_lds) atomicMax(&lds_amax[amax_idx - a_first], __float_as_uint(amax_chunk));
              else atomicMax(CODEC == KAON_MOM_INT8 ? &ws.ramax(T)[amax_idx] : &ws.bamax(T)[amax_idx],
                             __float_as_uint(amax_chunk));
            }
            amax_idx = idx;
            amax_chunk = 0.0f;
          }
          amax_chunk = fmaxf(amax_chunk, ax);
          // the element that starts a row/block copies its old scale
          if (CODEC == KAON_MOM_INT8) {
            if ((factored ? ji : e) == 0) ws.roldsc(T)[factored ? ri : 0] = rc.oldsc;
          } else if (e == blk * B) {
            ws.boldsc(T, nb)[blk] = b_oldsc;
          }
        }
      } else {
        // requant (_quant_int8 / _quant_4bit)
        float mdeq = 0.0f;
        if (quant) {
          if (CODEC == KAON_MOM_INT8) {
            float x = rintf(div_r64(mfv, rc.rnew));
            x = fminf(fmaxf(x, -127.0f), 127.0f);
            qout[i] = (uint32_t)(uint8_t)(int8_t)x;
            mdeq = x * rc.newsc;
            if ((factored ? ji : e) == 0) T.m_scale[factored ? ri : 0] = rc.newsc;
          } else {
            float x = rintf(div_r64(mfv, b_rnew));
            x = fminf(fmaxf(x, -7.0f), 7.0f);
            qout[i] = (uint32_t)((int)x + 8);
            mdeq = x * b_newsc;
            if (e == blk * B) T.m_scale[blk] = b_newsc;
          }
        } else if (mom) {
          mdeq = CODEC == KAON_MOM_BF16 ? bf2f(qout[i]) : __uint_as_float(qout[i]);
        }
        mnew[i] = mdeq;
        float dd = d;
        if (cautious) dd = div_r64(d * (kp ? 1.0f : 0.0f), rden);
        if (OPT == KAON_OPT_LION) dd = dd * hp.lr;
        dout[i] = dd;
        p[i] = pw;
      }
      // advance row/column of the next element
      if (factored && ++ji == C) {
        ji = 0;
        ++ri;
      }
    }

    if (PHASE == 5) {
      if (quant && amax_idx >= 0) {
        if (use_lds) atomicMax(&lds_amax[amax_idx - a_first], __float_as_uint(amax_chunk));
        else atomicMax(CODEC == KAON_MOM_INT8 ? &ws.ramax(T)[amax_idx] : &ws.bamax(T)[amax_idx],
                       __float_as_uint(amax_chunk));
      }
      continue;
    }

    // ---------------- phase 6 writes
    if (mom) st_mom_raw<CODEC>(T, e0, cnt, vec, qout);
    if (PT == KAON_F32) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x = p[i] - dout[i];
        if (nk_climb) x = x + msam_e(mnew[i] * (-hp.nk_k), hp.nk_bound_new);
        o[i] = x;
      }
      st8_f32(T.p, e0, cnt, vec, o);
    } else {
      uint32_t o[8];
      if (hp.bf16_method == KAON_KAHAN) {
        uint32_t sh[8];
        ld8_bits(T.shift, e0, cnt, vec, sh);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          // shift -= bf16(delta); p0 = p; p += shift; shift += p0 - p  (_backend.py:90-94)
          const float s = rbf(bf2f(sh[i]) - rbf(dout[i]));
          const float p0 = p[i];
          const float p1 = rbf(p0 + s);
          o[i] = f2bf(p1);
          sh[i] = f2bf(s + rbf(p0 - p1));
        }
        st8_bits(T.shift, e0, cnt, vec, sh);
      } else if (hp.bf16_method == KAON_RN) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = f2bf(p[i] - rbf(dout[i]));
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = sr_bf16(p[i] - dout[i], nz1[i]);
      }
      if (nk_climb) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          o[i] = sr_bf16(bf2f(o[i]) + msam_e(mnew[i] * (-hp.nk_k), hp.nk_bound_new), nz2[i]);
      }
      st8_bits(T.p, e0, cnt, vec, o);
    }
  }

  if (PHASE == 5) {
    if (cautious) {
      const uint32_t tot = wg_sum_u32(keep, lds4);
      if (threadIdx.x == 0 && tot) atomicAdd(&((uint32_t*)ws.scal(T))[1], tot);
    }
    if (quant && use_lds) {
      __syncthreads();
      for (int64_t a = a_first + threadIdx.x; a <= a_last; a += KAON_WG) {
        const uint32_t v = lds_amax[a - a_first];
        bool inside;
        if (CODEC == KAON_MOM_INT8) inside = !factored ? (e_begin == 0 && e_end == n)
                                                       : (a * C >= e_begin && (a + 1) * C <= e_end);
        else inside = a * B >= e_begin && min((a + 1) * B, n) <= e_end;
        uint32_t* dst = CODEC == KAON_MOM_INT8 ? &ws.ramax(T)[a] : &ws.bamax(T)[a];
        if (inside) *dst = v;
        else atomicMax(dst, v);
      }
    }
  }
}

// =============================================================== MSAM apply
template <int PT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_msam(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, KaonHyper hp,
                                                  float factor, float bound, uint32_t sid) {
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C;
  const int64_t e_begin = it.row0, e_end = (int64_t)it.row0 + it.nrows;
  const bool vecT = T.vec_flat != 0;
  for (int64_t e0 = e_begin + 8 * (int64_t)threadIdx.x; e0 < e_end; e0 += 8 * KAON_WG) {
    const int cnt = (int)min<int64_t>(8, e_end - e0);
    const bool vec = vecT && cnt == 8;
    uint32_t mq[8];
    ld_mom_raw<CODEC>(T, e0, cnt, vec, mq);
    float ev[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t e = e0 + i;
      float mold = 0.0f;
      if (i < cnt) {
        if (CODEC == KAON_MOM_INT8) mold = (float)(int8_t)(uint8_t)mq[i] * T.m_scale[T.factored ? e / C : 0];
        else if (CODEC == KAON_MOM_4BIT) mold = ((float)mq[i] - 8.0f) * T.m_scale[e / T.block4];
        else if (CODEC == KAON_MOM_BF16) mold = bf2f(mq[i]);
        else mold = __uint_as_float(mq[i]);
      }
      ev[i] = msam_e(mold * factor, bound);
    }
    if (PT == KAON_F32) {
      float p[8];
      ld8<KAON_F32>(T.p, e0, cnt, vec, p);
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = p[i] + ev[i];
      st8_f32(T.p, e0, cnt, vec, p);
    } else {
      uint32_t pb[8], nz[8];
      ld8_bits(T.p, e0, cnt, vec, pb);
      noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, sid, e0, T.noise[sid], cnt, nz);
#pragma unroll
      for (int i = 0; i < 8; ++i) pb[i] = sr_bf16(bf2f(pb[i]) + ev[i], nz[i]);
      st8_bits(T.p, e0, cnt, vec, pb);
    }
  }
}

// =============================================================== primitives
__global__ void k_quant_int8(const float* __restrict__ m, int64_t rows, int64_t cols, int8_t* __restrict__ q,
                             float* __restrict__ scale) {
  __shared__ float red[KAON_WG];
  const int64_t r = blockIdx.x;
  if (r >= rows) return;
  const float* x = m + r * cols;
  float a = 0.0f;
  for (int64_t j = threadIdx.x; j < cols; j += KAON_WG) a = fmaxf(a, fabsf(x[j]));
  red[threadIdx.x] = a;
  __syncthreads();
  for (int o = KAON_WG / 2; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  const float sc = fmaxf(red[0], 1e-12f) / 127.0f;
  const double rs = rcp64(sc);
  for (int64_t j = threadIdx.x; j < cols; j += KAON_WG) {
    float v = rintf(div_r64(x[j], rs));
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    q[r * cols + j] = (int8_t)v;
  }
  if (threadIdx.x == 0) scale[r] = sc;
}

__global__ void k_quant_4bit_scale(const float* __restrict__ m, int64_t n, int32_t block, float* __restrict__ scale) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nb = (n + block - 1) / block;
  if (b >= nb) return;
  float a = 0.0f;
  for (int64_t i = b * block; i < min<int64_t>((b + 1) * block, n); ++i) a = fmaxf(a, fabsf(m[i]));
  scale[b] = fmaxf(a, 1e-12f) / 7.0f;
}

__global__ void k_quant_4bit_pack(const float* __restrict__ m, int64_t n, int32_t block,
                                  const float* __restrict__ scale, uint8_t* __restrict__ packed) {
  const int64_t byte = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (2 * byte >= n) return;
  uint32_t out = 0;
  for (int h = 0; h < 2; ++h) {
    const int64_t i = 2 * byte + h;
    if (i >= n) break;
    float x = rintf(div_r64(m[i], rcp64(scale[i / block])));
    x = fminf(fmaxf(x, -7.0f), 7.0f);
    out |= (uint32_t)((int)x + 8) << (4 * h);
  }
  packed[byte] = (uint8_t)out;
}

__global__ void k_dequant(int32_t codec, const void* __restrict__ m, const float* __restrict__ scale, int64_t rows,
                          int64_t cols, int32_t block, float* __restrict__ out) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float v = 0.0f;
    if (codec == KAON_MOM_INT8) v = (float)((const int8_t*)m)[i] * scale[i / cols];
    else if (codec == KAON_MOM_4BIT) {
      const uint32_t b = ((const uint8_t*)m)[i >> 1];
      v = ((float)((b >> (4 * (i & 1))) & 0xFu) - 8.0f) * scale[i / block];
    } else if (codec == KAON_MOM_BF16) v = bf2f(((const uint16_t*)m)[i]);
    else if (codec == KAON_MOM_F32) v = ((const float*)m)[i];
    out[i] = v;
  }
}

__global__ void k_sr_round(const float* __restrict__ x, const uint16_t* __restrict__ noise, int64_t n,
                           uint16_t* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = (uint16_t)sr_bf16(x[i], noise[i]);
}

__global__ void k_sr_noise(uint16_t* __restrict__ out, int64_t n, uint64_t seed, uint32_t step, uint32_t tid,
                           uint32_t sid) {
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c * 8 < n; c += (int64_t)gridDim.x * blockDim.x) {
    uint32_t w[8];
    const int cnt = (int)min<int64_t>(8, n - c * 8);
    noise8(seed, step, tid, sid, c * 8, nullptr, cnt, w);
    for (int i = 0; i < cnt; ++i) out[c * 8 + i] = (uint16_t)w[i];
  }
}

__global__ __launch_bounds__(KAON_WG) void k_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    dst[i] = a;
    dst[i + stride] = b;
    dst[i + 2 * stride] = c;
    dst[i + 3 * stride] = d;
  }
  for (; i < n16; i += stride) dst[i] = src[i];
}

// ------------------------------------------------------------ dispatch tables
using FlatFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper);

template <int OPT, int PHASE, int PT, int GT>
FlatFn flat_by_codec(int codec) {
  switch (codec) {
    case KAON_MOM_NONE: return k_flat<OPT, PHASE, PT, GT, KAON_MOM_NONE>;
    case KAON_MOM_F32: return k_flat<OPT, PHASE, PT, GT, KAON_MOM_F32>;
    case KAON_MOM_BF16: return k_flat<OPT, PHASE, PT, GT, KAON_MOM_BF16>;
    case KAON_MOM_INT8: return k_flat<OPT, PHASE, PT, GT, KAON_MOM_INT8>;
    case KAON_MOM_4BIT: return k_flat<OPT, PHASE, PT, GT, KAON_MOM_4BIT>;
  }
  return nullptr;
}

template <int OPT, int PHASE>
FlatFn flat_fn(int pt, int gt, int codec) {
  if (pt == KAON_BF16 && gt == KAON_BF16) return flat_by_codec<OPT, PHASE, KAON_BF16, KAON_BF16>(codec);
  if (pt == KAON_BF16 && gt == KAON_F32) return flat_by_codec<OPT, PHASE, KAON_BF16, KAON_F32>(codec);
  if (pt == KAON_F32 && gt == KAON_BF16) return flat_by_codec<OPT, PHASE, KAON_F32, KAON_BF16>(codec);
  if (pt == KAON_F32 && gt == KAON_F32) return flat_by_codec<OPT, PHASE, KAON_F32, KAON_F32>(codec);
  return nullptr;
}

using RowsFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper, int);
template <int GT>
RowsFn rows_fn_gt(int km) {
  switch (km) {
    case 1: return k_rows<GT, 1>;
    case 2: return k_rows<GT, 2>;
    case 4: return k_rows<GT, 4>;
    case 8: return k_rows<GT, 8>;
  }
  return nullptr;
}
RowsFn rows_fn(int gt, int km) { return gt == KAON_BF16 ? rows_fn_gt<KAON_BF16>(km) : rows_fn_gt<KAON_F32>(km); }

using MsamFn = void (*)(const KaonTensor*, const KaonItem*, KaonHyper, float, float, uint32_t);
MsamFn msam_fn(int pt, int codec) {
#define KAON_MSAM_CASE(PTV)                                            \
  switch (codec) {                                                     \
    case KAON_MOM_F32: return k_msam<PTV, KAON_MOM_F32>;               \
    case KAON_MOM_BF16: return k_msam<PTV, KAON_MOM_BF16>;             \
    case KAON_MOM_INT8: return k_msam<PTV, KAON_MOM_INT8>;             \
    case KAON_MOM_4BIT: return k_msam<PTV, KAON_MOM_4BIT>;             \
  }
  if (pt == KAON_BF16) { KAON_MSAM_CASE(KAON_BF16) }
  else { KAON_MSAM_CASE(KAON_F32) }
#undef KAON_MSAM_CASE
  return nullptr;
}

using SsFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper);
SsFn ss_fn(int gt) { return gt == KAON_BF16 ? (SsFn)k_ss<KAON_BF16> : (SsFn)k_ss<KAON_F32>; }

// Phase-1 launches, one per register class run (items are sorted by class).
int launch_rows(const KaonLaunch& L, Ws ws, const KaonHyper& hp, int mode, hipStream_t st) {
  int32_t off = 0;
  for (int cls = 0; cls < 4; ++cls) {
    const int32_t cnt = L.row_runs[cls];
    if (cnt <= 0) continue;
    RowsFn fn = rows_fn(hp.g_dtype, 1 << cls);
    hipLaunchKernelGGL(fn, dim3(cnt), dim3(KAON_WG), 0, st, L.descs, L.row_items + off, ws, hp, mode);
    off += cnt;
  }
  if (off != L.n_row_items) return fail("kaon: row-item class runs do not add up to n_row_items");
  return check_launch("kaon: k_rows launch");
}

int validate(const KaonLaunch* L, const KaonHyper* hp, const char* who) {
  if (!L || !hp) return fail(who);
  if (hp->p_dtype != KAON_F32 && hp->p_dtype != KAON_BF16) return fail("kaon: bad p_dtype");
  if (hp->g_dtype != KAON_F32 && hp->g_dtype != KAON_BF16) return fail("kaon: bad g_dtype");
  if (hp->codec < KAON_MOM_NONE || hp->codec > KAON_MOM_4BIT) return fail("kaon: bad codec");
  if (hp->bf16_method < KAON_SR || hp->bf16_method > KAON_KAHAN) return fail("kaon: bad bf16_method");
  if (L->n_tensors > 0 && (!L->descs || !L->workspace)) return fail("kaon: null descriptor table or workspace");
  return 0;
}

}  // namespace

// ====================================================================== C ABI
extern "C" {

int kaon_abi_version(void) { return KAON_ABI_VERSION; }

const char* kaon_last_error(void) { return g_err.c_str(); }

int kaon_adakaon_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream) {
  int rc = validate(L, hp, "kaon_adakaon_phases: null argument");
  if (rc) return rc;
  if (L->n_tensors <= 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  const bool mom = (h.flags & KAON_F_MOMENTUM) && h.codec != KAON_MOM_NONE;
  const int codec = mom ? h.codec : KAON_MOM_NONE;
  if (!mom) h.flags &= ~(KAON_F_MOMENTUM | KAON_F_NK_REMOVE | KAON_F_NK_CLIMB);
  const bool quant = codec == KAON_MOM_INT8 || codec == KAON_MOM_4BIT;
  if (mask & (1u << 1)) {
    if ((rc = launch_rows(*L, ws, h, 0, st))) return rc;
  }
  if ((mask & (1u << 2)) && L->n_fin_items > 0) {
    hipLaunchKernelGGL(k_fin, dim3(L->n_fin_items), dim3(KAON_WG), 0, st, L->descs, L->fin_items, ws, h);
    if ((rc = check_launch("kaon: k_fin launch"))) return rc;
  }
  if (mask & (1u << 3)) {
    hipLaunchKernelGGL(ss_fn(h.g_dtype), dim3(L->n_row_items), dim3(KAON_WG), 0, st, L->descs, L->row_items, ws,
                       h);
    if ((rc = check_launch("kaon: k_ss launch"))) return rc;
  }
  if (mask & (1u << 4)) {
    hipLaunchKernelGGL(k_fac, dim3(L->n_tensors), dim3(KAON_WG), 0, st, L->descs, ws, h);
    if ((rc = check_launch("kaon: k_fac launch"))) return rc;
  }
  if ((mask & (1u << 5)) && ((h.flags & KAON_F_CAUTIOUS) || quant)) {
    FlatFn f5 = flat_fn<KAON_OPT_ADAKAON, 5>(h.p_dtype, h.g_dtype, codec);
    hipLaunchKernelGGL(f5, dim3(L->n_flat_items), dim3(KAON_WG), 0, st, L->descs, L->flat_items, ws, h);
    if ((rc = check_launch("kaon: keep-count launch"))) return rc;
  }
  if (mask & (1u << 6)) {
    FlatFn f6 = flat_fn<KAON_OPT_ADAKAON, 6>(h.p_dtype, h.g_dtype, codec);
    hipLaunchKernelGGL(f6, dim3(L->n_flat_items), dim3(KAON_WG), 0, st, L->descs, L->flat_items, ws, h);
    if ((rc = check_launch("kaon: apply launch"))) return rc;
  }
  return 0;
}

int kaon_adakaon_step(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  return kaon_adakaon_phases(L, hp, 0x7Eu, stream);
}

int kaon_lion_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream) {
  int rc = validate(L, hp, "kaon_lion_phases: null argument");
  if (rc) return rc;
  if (L->n_tensors <= 0) return 0;
  if (hp->codec == KAON_MOM_NONE) return fail("kaon_lion_step: Lion always keeps a momentum buffer");
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  h.flags |= KAON_F_MOMENTUM;
  h.flags &= ~(KAON_F_NK_REMOVE | KAON_F_NK_CLIMB);
  const bool quant = h.codec == KAON_MOM_INT8 || h.codec == KAON_MOM_4BIT;
  if (mask & (1u << 1)) {
    if ((rc = launch_rows(*L, ws, h, 1, st))) return rc;
  }
  if ((mask & (1u << 5)) && ((h.flags & KAON_F_CAUTIOUS) || quant)) {
    FlatFn f5 = flat_fn<KAON_OPT_LION, 5>(h.p_dtype, h.g_dtype, h.codec);
    hipLaunchKernelGGL(f5, dim3(L->n_flat_items), dim3(KAON_WG), 0, st, L->descs, L->flat_items, ws, h);
    if ((rc = check_launch("kaon: lion keep-count launch"))) return rc;
  }
  if (mask & (1u << 6)) {
    FlatFn f6 = flat_fn<KAON_OPT_LION, 6>(h.p_dtype, h.g_dtype, h.codec);
    hipLaunchKernelGGL(f6, dim3(L->n_flat_items), dim3(KAON_WG), 0, st, L->descs, L->flat_items, ws, h);
    if ((rc = check_launch("kaon: lion apply launch"))) return rc;
  }
  return 0;
}

int kaon_lion_step(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  return kaon_lion_phases(L, hp, 0x62u, stream);
}

int kaon_msam_apply(const KaonLaunch* L, const KaonHyper* hp, float factor, float bound, uint32_t stream_id,
                    void* stream) {
  int rc = validate(L, hp, "kaon_msam_apply: null argument");
  if (rc) return rc;
  if (L->n_tensors <= 0) return 0;
  if (stream_id > 2) return fail("kaon_msam_apply: stream_id must be 0, 1 or 2");
  MsamFn fn = msam_fn(hp->p_dtype, hp->codec);
  if (!fn) return fail("kaon_msam_apply: needs a momentum codec");
  hipLaunchKernelGGL(fn, dim3(L->n_flat_items), dim3(KAON_WG), 0, (hipStream_t)stream, L->descs, L->flat_items,
                     *hp, factor, bound, stream_id);
  return check_launch("kaon: msam launch");
}

// ---------------------------------------------------------------- primitives
static unsigned grid_for(int64_t n, int per_thread) {
  int64_t g = (n + (int64_t)KAON_WG * per_thread - 1) / ((int64_t)KAON_WG * per_thread);
  if (g < 1) g = 1;
  if (g > 65535) g = 65535;
  return (unsigned)g;
}

int kaon_quant_int8(const float* m, int64_t rows, int64_t cols, int8_t* q, float* scale, void* stream) {
  if (rows <= 0 || cols <= 0) return 0;
  if (rows > 0x7FFFFFFF) return fail("kaon_quant_int8: too many rows");
  hipLaunchKernelGGL(k_quant_int8, dim3((unsigned)rows), dim3(KAON_WG), 0, (hipStream_t)stream, m, rows, cols, q, scale);
  return check_launch("kaon_quant_int8");
}

int kaon_quant_4bit(const float* m, int64_t n, int32_t block, uint8_t* packed, float* scale, void* stream) {
  if (n <= 0) return 0;
  if (block <= 0) return fail("kaon_quant_4bit: block must be > 0");
  const int64_t nb = (n + block - 1) / block;
  hipLaunchKernelGGL(k_quant_4bit_scale, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, (hipStream_t)stream, m, n,
                     block, scale);
  const int64_t nbytes = (n + 1) / 2;
  hipLaunchKernelGGL(k_quant_4bit_pack, dim3((unsigned)((nbytes + 255) / 256)), dim3(256), 0, (hipStream_t)stream, m,
                     n, block, scale, packed);
  return check_launch("kaon_quant_4bit");
}

int kaon_dequant(int32_t codec, const void* m, const float* scale, int64_t rows, int64_t cols, int32_t block,
                 float* out, void* stream) {
  if (rows <= 0 || cols <= 0) return 0;
  if (codec == KAON_MOM_4BIT && block <= 0) return fail("kaon_dequant: block must be > 0");
  hipLaunchKernelGGL(k_dequant, dim3(grid_for(rows * cols, 1)), dim3(KAON_WG), 0, (hipStream_t)stream, codec, m,
                     scale, rows, cols, block, out);
  return check_launch("kaon_dequant");
}

int kaon_sr_round(const float* x, const uint16_t* noise, int64_t n, uint16_t* out, void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_sr_round, dim3(grid_for(n, 4)), dim3(KAON_WG), 0, (hipStream_t)stream, x, noise, n, out);
  return check_launch("kaon_sr_round");
}

int kaon_sr_noise(uint16_t* out, int64_t n, uint64_t seed, uint32_t step, uint32_t tensor_id, uint32_t stream_id,
                  void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_sr_noise, dim3(grid_for((n + 7) / 8, 1)), dim3(KAON_WG), 0, (hipStream_t)stream, out, n, seed,
                     step, tensor_id, stream_id);
  return check_launch("kaon_sr_noise");
}

int kaon_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (bytes <= 0) return 0;
  if ((bytes & 15) || (((uintptr_t)src | (uintptr_t)dst) & 15)) return fail("kaon_copy: needs 16-byte alignment");
  const int64_t n16 = bytes / 16;
  int64_t g = (n16 + KAON_WG * 4 - 1) / (KAON_WG * 4);
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(k_copy, dim3((unsigned)g), dim3(KAON_WG), 0, (hipStream_t)stream, (const uint4*)src, (uint4*)dst,
                     n16);
  return check_launch("kaon_copy");
}

}  // extern "C"
