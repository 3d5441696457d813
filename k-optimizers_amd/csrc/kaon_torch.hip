// kaon_torch.hip -- the step's fp32 sums in torch CPU's order (KAON_F_TORCH_ORDER).
//
// The canonical step sums in a fixed 64-lane order.  torch fixes no order of its
// own, but the reference's results are those of torch 2.10 on x86-64, whose CPU
// kernels sum in a definite order (measured against torch, restated in
// oracle/kaon_oracle.c: torch_msum, ko_torch_inner_sum, ko_torch_outer_sum,
// ko_torch_sumsq).  This opt-in mode computes the five sums of a step in that
// order, so the HIP step gives the reference's weights bit for bit:
//
//  * the GC row mean of the gradient (centralize_grads_, _backend.py:147-177:
//    torch's mean over dims 1.., one rounding of fp32 sum / C to the grad dtype);
//  * the factored row means mean_C(G^2 + eps1) (_factored.py:51);
//  * the column means mean_R(G^2 + eps1) (_factored.py:52);
//  * the mean of the row EMA behind the row factors (_factored.py:76-82);
//  * ||U||, the RMS clip's norm (_backend.py:45-47 at adakaon.py:1001): eight
//    sequential fused multiply-add chains;
//  * MSAM norm="tensor"'s per-tensor sum of the squared momentum (msam.py:219-221).
//
// Phases 5 and 6 then run unchanged on what these kernels leave in the
// workspace (GC means, row factors, column factors, the clip divisor).
//
// Cascade sums are parallel over accumulator positions (32 of a row's, one per
// column) and sequential inside each, as torch's are.  The clip norm's chains
// are inherently sequential: one workgroup per tensor, three waves computing U
// a block ahead into LDS, eight lanes of the fourth running the chains.
#include "kaon_common.h"

namespace kaon {

namespace {

__device__ __forceinline__ int ceil_log2_u64(uint64_t x) { return x > 1 ? 64 - __clzll((long long)(x - 1)) : 0; }

// One accumulator position of torch_msum's cascade over `size` terms term(0..size-1),
// run by one lane: level 0 sums a leaf of 2^lp terms from 0, lp = max(4,
// ceil(log2(size)) / 4); each finished leaf goes into level 1, which goes into
// level 2 every 2^lp leaves, which goes into level 3 every 2^(2 lp) leaves;
// leftover terms go into level 0, and the levels are added 0 + 1, + 2, + 3.
template <class F>
__device__ float tcascade(int64_t size, F term) {
  const int lp0 = ceil_log2_u64((uint64_t)size) / 4;
  const int lp = lp0 > 4 ? lp0 : 4;
  const int64_t step = (int64_t)1 << lp, mask = step - 1;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  int64_t i = 0;
  while (i + step <= size) {
    if (lp == 4) {
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = term(i + j);
#pragma unroll
      for (int j = 0; j < 16; ++j) a0 = a0 + v[j];
    } else {
      for (int64_t j = 0; j < step; ++j) a0 = a0 + term(i + j);
    }
    i += step;
    a1 = a1 + a0;
    a0 = 0.0f;
    if ((i & (mask << lp)) == 0) {
      a2 = a2 + a1;
      a1 = 0.0f;
      if ((i & (mask << (2 * lp))) == 0) {
        a3 = a3 + a2;
        a2 = 0.0f;
      }
    }
  }
  for (; i < size; ++i) a0 = a0 + term(i);
  a0 = a0 + a1;
  a0 = a0 + a2;
  a0 = a0 + a3;
  return a0;
}

// torch's sum of a contiguous row of n fp32 terms ld(0..n-1) (ko_torch_inner_sum),
// by the 32 lanes of a half-wave, pos = lane % 32.  Rows of 8 or more: position
// pos = 8 k + l is slot k, lane l of the 8-float vectors, a cascade over the
// n / 32 rows of four vectors; the leftover vectors go into slot 0, slots 1-3 are
// added into slot 0 in order, then the scalar tail and the 8 lanes are added in
// order from 0.  Shorter rows: four single-term slots over n / 4 rows, every
// lane computing the same.  Call with the whole wave active (the exchanges read
// other lanes); every lane of the half returns the sum.
template <class F>
__device__ float tinner32(int64_t n, int pos, F ld) {
  if (n < 8) {
    const int64_t size = n / 4;
    float ps[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) ps[k] = tcascade(size, [&](int64_t i) { return ld(4 * i + k); });
    for (int64_t i = 4 * size; i < n; ++i) ps[0] = ps[0] + ld(i);
    return ((ps[0] + ps[1]) + ps[2]) + ps[3];
  }
  const int base = (int)(threadIdx.x & 32);
  const int64_t nv = n / 8, size = nv / 4;
  float acc = tcascade(size, [&](int64_t i) { return ld(32 * i + pos); });
  if (pos < 8)
    for (int64_t v = 4 * size; v < nv; ++v) acc = acc + ld(8 * v + pos);
  const float s1 = __shfl(acc, base + ((pos + 8) & 31));
  const float s2 = __shfl(acc, base + ((pos + 16) & 31));
  const float s3 = __shfl(acc, base + ((pos + 24) & 31));
  acc = ((acc + s1) + s2) + s3;
  float f = 0.0f;
  for (int64_t k = 8 * nv; k < n; ++k) f = f + ld(k);
#pragma unroll
  for (int l = 0; l < 8; ++l) f = f + __shfl(acc, base + l);
  return f;
}

// Element j of a grad / source row as fp32.
template <int GT>
__device__ __forceinline__ float ldx(const void* base, int64_t j) {
  if (GT == KAON_F32) return G((const float*)base)[j];
  return lp2f<GT>(G((const uint16_t*)base)[j]);
}

// =============================================================== phase 1
// Runs (row items): the GC mean and the row EMA of every row in torch's order;
// 1-D tensors: the elementwise v EMA.  The two halves of each wave take two
// rows.  mode 1 (Lion): GC means only.
template <int GT>
__global__ __launch_bounds__(KAON_WG) void k_trow(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws, KaonHyper hp,
                                                  int mode) {
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  zero_accumulators(T, it, ws, hp.codec);
  const void* gsrc = T.g;
  if (!T.factored) {
    if (mode == 0) stats_1d<GT>(T, gsrc, hp);
    return;
  }
  const bool gc = (hp.flags & KAON_F_GC) != 0;
  if (mode == 1 && !gc) return;
  const bool eps = (hp.flags & KAON_F_EPS) != 0;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = (int)(threadIdx.x & 63), half = lane >> 5, pos = lane & 31;
  const int64_t C = T.C, end = (int64_t)it.row0 + it.nrows;
  for (int64_t rb = (int64_t)it.row0 + 2 * w; rb < end; rb += 8) {
    // a half without a row of its own repeats the last one and stores nothing
    const bool own = rb + half < end;
    const int64_t r = own ? rb + half : end - 1;
    const int64_t off = r * C;
    float mu = 0.0f;
    if (gc) {
      const float s = tinner32(C, pos, [&](int64_t j) { return ldx<GT>(gsrc, off + j); });
      mu = round_to<GT>(s / (float)C);
      if (own && pos == 0) ws.mu(T)[r] = mu;
    }
    if (mode == 1) continue;
    const float s2 = tinner32(C, pos, [&](int64_t j) {
      float x = ldx<GT>(gsrc, off + j);
      if (gc) x = round_to<GT>(x - mu);
      float q = x * x;
      if (eps) q = q + hp.eps1;
      return q;
    });
    if (own && pos == 0) G(T.row)[r] = klerp(G(T.row)[r], s2 / (float)C, hp.w2);
  }
}

// =============================================================== phase 2
// Finalize items, eight workgroups each.  kind 0: columns [row0, row0 + nrows),
// 256 per workgroup, one per thread: the column sum of G^2 (+eps1) over the rows
// (ko_torch_outer_sum: a cascade down the rows for the blocks of 32 columns --
// blocks of 4 when C < 8 -- and four row slots for the columns after them), then
// col = lerp(col, sum / R, 1-beta2) and cf = 1/sqrt(col).  kind 1: the row EMA's
// mean in torch's row order, rf = 1/sqrt(row / mean).
constexpr int kTfinSub = 8;

template <int GT>
__global__ __launch_bounds__(KAON_WG) void k_tfin(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ float rm_s;
  const KaonItem it = items[blockIdx.x / kTfinSub];
  const int sb = (int)(blockIdx.x % kTfinSub);
  const KaonTensor& T = D[it.tensor];
  const int64_t R = T.R, C = T.C;
  if (it.kind == 0) {
    const int64_t j = (int64_t)it.row0 + (int64_t)sb * KAON_WG + threadIdx.x;
    if (j >= (int64_t)it.row0 + it.nrows) return;
    const void* gsrc = T.g;
    const bool gc = (hp.flags & KAON_F_GC) != 0;
    const bool eps = (hp.flags & KAON_F_EPS) != 0;
    const KAON_G float* mu = ws.mu(T);
    auto q = [&](int64_t i) {
      float x = ldx<GT>(gsrc, i * C + j);
      if (gc) x = round_to<GT>(x - mu[i]);
      float v = x * x;
      if (eps) v = v + hp.eps1;
      return v;
    };
    const int64_t jd = C >= 8 ? (C / 32) * 32 : (C / 4) * 4;
    float cs;
    if (j < jd) {
      cs = tcascade(R, q);
    } else {
      const int64_t size = R / 4;
      float ps[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) ps[k] = tcascade(size, [&](int64_t i) { return q(4 * i + k); });
      for (int64_t i = 4 * size; i < R; ++i) ps[0] = ps[0] + q(i);
      cs = ((ps[0] + ps[1]) + ps[2]) + ps[3];
    }
    const float nc = klerp(G(T.col)[j], cs / (float)R, hp.w2);
    G(T.col)[j] = nc;
    ws.cf(T)[j] = 1.0f / sqrtf(nc);
  } else {
    if (sb != 0) return;
    const KAON_G float* row = G((const float*)T.row);
    if (threadIdx.x < 64) {
      const float s = tinner32(R, (int)(threadIdx.x & 31), [&](int64_t i) { return row[i]; });
      if (threadIdx.x == 0) rm_s = s / (float)R;
    }
    __syncthreads();
    const float rm = rm_s;
    KAON_G float* rf = ws.rf(T);
    for (int64_t i = threadIdx.x; i < R; i += KAON_WG) rf[i] = 1.0f / sqrtf(row[i] / rm);
  }
}

// =============================================================== phases 3-4
// The clip divisor max(||U|| / sqrt(n) / clip, 1) of each tensor (one workgroup
// per tensor), ||U||^2 as torch's norm kernel forms it: lane k of 8 a sequential
// fma chain over elements k, k+8, ... of the first n - n % 8, the 8 lanes added
// in order, the tail fma'd after.  U = (G' r) c (factored) or g / sqrt(v) (1-D),
// G' the GC'd gradient.  Blocks of kTcS chunks of 8 elements: waves 1-3 compute
// U of block b + 1 into one LDS buffer (chunk s of the block -> column s, element
// k -> row k) while lanes 0-7 of wave 0 run the chains over block b in the other.
constexpr int kTcS = 896;                  // chunks (chain steps) per block
constexpr int kTcLd = kTcS + 4;            // LDS row stride: the 8 chain rows fall in distinct banks
constexpr int kTcProd = KAON_WG - 64;      // producer threads
constexpr int kTcSlots = (kTcS + kTcProd - 1) / kTcProd;

// U of element e (the tail and ragged rows).
template <int GT>
__device__ __forceinline__ float tclip_u(const KaonTensor& T, const Ws& ws, bool gc, int64_t e) {
  const float x = ldx<GT>(T.g, e);
  if (!T.factored) return x * (1.0f / sqrtf(G(T.v)[e]));
  const uint32_t r = (uint32_t)e / (uint32_t)T.C, j = (uint32_t)e - r * (uint32_t)T.C;
  const float xg = gc ? round_to<GT>(x - ws.mu(T)[r]) : x;
  return (xg * ws.rf(T)[r]) * ws.cf(T)[j];
}

template <int GT>
__global__ __launch_bounds__(KAON_WG) void k_tclip(const KaonTensor* __restrict__ D, int32_t n_tensors, Ws ws,
                                                   KaonHyper hp) {
  __shared__ __align__(16) float lds[2 * 8 * kTcLd];
  const int t = (int)blockIdx.x;
  if (t >= n_tensors) return;
  const KaonTensor& T = D[t];
  const int64_t n = T.n;
  if (n == 0) return;
  const bool gc = (hp.flags & KAON_F_GC) != 0 && T.factored;
  const int64_t body = n - n % 8, nchunks = body / 8;
  const int64_t nblk = (nchunks + kTcS - 1) / kTcS;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = (int)(threadIdx.x & 63);
  // chunk kinds: 0 = 1-D, 1 = factored rows of whole chunks, 2 = chunks across rows
  const int kind = !T.factored ? 0 : (T.C % 8 == 0 ? 1 : 2);
  const bool vec = T.vec_rows != 0;
  const uint32_t cpr = (uint32_t)(T.C / 8);

  auto produce = [&](int64_t b, int buf) {
    const int q0 = (int)threadIdx.x - 64;
    float x[kTcSlots][8], f[kTcSlots][8], mu[kTcSlots], rf[kTcSlots];
    // every load of the block's slots first, then the arithmetic
#pragma unroll
    for (int k = 0; k < kTcSlots; ++k) {
      const int s = q0 + kTcProd * k;
      const int64_t c = b * kTcS + s;
      mu[k] = 0.0f;
      rf[k] = 1.0f;
      if (s >= kTcS || c >= nchunks) continue;
      if (kind == 0) {
        ld8<GT>(T.g, c * 8, 8, vec, x[k]);
        ld8<KAON_F32>(T.v, c * 8, 8, vec, f[k]);
      } else if (kind == 1) {
        const uint32_t r = (uint32_t)c / cpr, j0 = ((uint32_t)c - r * cpr) * 8u;
        ld8<GT>(T.g, c * 8, 8, vec, x[k]);
        ld8<KAON_F32>((const float*)ws.cf(T), j0, 8, vec, f[k]);
        if (gc) mu[k] = ws.mu(T)[r];
        rf[k] = ws.rf(T)[r];
      }
    }
#pragma unroll
    for (int k = 0; k < kTcSlots; ++k) {
      const int s = q0 + kTcProd * k;
      if (s >= kTcS) continue;
      const int64_t c = b * kTcS + s;
      float u[8];
      if (c >= nchunks) {
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = 0.0f;
      } else if (kind == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = x[k][i] * (1.0f / sqrtf(f[k][i]));
      } else if (kind == 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xg = gc ? round_to<GT>(x[k][i] - mu[k]) : x[k][i];
          u[i] = (xg * rf[k]) * f[k][i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = tclip_u<GT>(T, ws, gc, c * 8 + i);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) lds[(buf * 8 + i) * kTcLd + s] = u[i];
    }
  };

  if (wave != 0 && nblk > 0) produce(0, 0);
  __syncthreads();
  float acc = 0.0f;  // lane k < 8: chain k
  for (int64_t b = 0; b < nblk; ++b) {
    if (wave == 0) {
      if (lane < 8) {
        const int cnt = (int)min<int64_t>(kTcS, nchunks - b * kTcS);
        const float* row = lds + ((int)(b & 1) * 8 + lane) * kTcLd;
        int s = 0;
#pragma unroll 4
        for (; s + 4 <= cnt; s += 4) {
          const kf4 v = *(const kf4*)(row + s);
          acc = __fmaf_rn(v.x, v.x, acc);
          acc = __fmaf_rn(v.y, v.y, acc);
          acc = __fmaf_rn(v.z, v.z, acc);
          acc = __fmaf_rn(v.w, v.w, acc);
        }
        for (; s < cnt; ++s) acc = __fmaf_rn(row[s], row[s], acc);
      }
    } else if (b + 1 < nblk) {
      produce(b + 1, (int)((b + 1) & 1));
    }
    __syncthreads();
  }
  if (wave != 0) return;
  float ss = __shfl(acc, 0);
#pragma unroll
  for (int k = 1; k < 8; ++k) ss = ss + __shfl(acc, k);
  for (int64_t e = body; e < n; ++e) {
    const float u = tclip_u<GT>(T, ws, gc, e);
    ss = __fmaf_rn(u, u, ss);
  }
  // clip_threshold 0 leaves the update unclipped
  if (lane == 0) ws.scal(T)[0] = hp.clip > 0.0f ? fmaxf((sqrtf(ss) / T.sqrt_n) / hp.clip, 1.0f) : 1.0f;
}

// =============================================================== MSAM norm="tensor"
// Each tensor's sum of its squared dequantized momentum, (m * m).reshape(n,
// -1).sum(dim=1) (msam.py:219-221): one contiguous row of n terms in torch's row
// order, into the tensor's scalar word 2.  One workgroup per tensor, wave 0.
template <int CODEC>
__device__ __forceinline__ float mom_at(const KaonTensor& T, int64_t e) {
  if (CODEC == KAON_MOM_F32) return G((const float*)T.m)[e];
  if (CODEC == KAON_MOM_BF16) return bf2f(G((const uint16_t*)T.m)[e]);
  if (CODEC == KAON_MOM_INT8) {
    const uint32_t r = T.factored ? (uint32_t)e / (uint32_t)T.C : 0u;
    return (float)G((const int8_t*)T.m)[e] * G(T.m_scale)[r];
  }
  const uint8_t byte = G((const uint8_t*)T.m)[e >> 1];
  const uint32_t nib = (e & 1) ? (uint32_t)(byte >> 4) : (uint32_t)(byte & 15u);
  return ((float)nib - 8.0f) * G(T.m_scale)[(uint32_t)e / (uint32_t)T.block4];
}

template <int CODEC>
__global__ __launch_bounds__(64) void k_tmsq(const KaonTensor* __restrict__ D, int32_t n_tensors, Ws ws) {
  const int t = (int)blockIdx.x;
  if (t >= n_tensors) return;
  const KaonTensor& T = D[t];
  const float s = tinner32(T.n, (int)(threadIdx.x & 31), [&](int64_t e) {
    const float m = mom_at<CODEC>(T, e);
    return m * m;
  });
  if (threadIdx.x == 0) ws.scal(T)[2] = s;
}

using TrowFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper, int);
using TfinFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper);
using TclipFn = void (*)(const KaonTensor*, int32_t, Ws, KaonHyper);

}  // namespace

// Phases 1-4 of an Adakaon step (mode 0) or phase 1 of a Lion step (mode 1) in
// torch's order, for the phase bits of `mask` (1, 2, 3; phase 3 also leaves the
// clip divisor, so bit 4 has nothing left to do).  Returns a HIP status.
int torch_phases(const KaonLaunch& L, Ws ws, const KaonHyper& h, uint32_t mask, int mode, hipStream_t st) {
  const int gt = h.g_dtype;
  if (mask & (1u << 1)) {
    TrowFn f = gt == KAON_BF16 ? k_trow<KAON_BF16> : gt == KAON_F16 ? k_trow<KAON_F16> : k_trow<KAON_F32>;
    hipLaunchKernelGGL(f, dim3(L.n_row_items), dim3(KAON_WG), 0, st, L.descs, L.row_items, ws, h, mode);
  }
  if (mode == 0 && (mask & (1u << 2)) && L.n_fin_items > 0) {
    TfinFn f = gt == KAON_BF16 ? k_tfin<KAON_BF16> : gt == KAON_F16 ? k_tfin<KAON_F16> : k_tfin<KAON_F32>;
    hipLaunchKernelGGL(f, dim3(L.n_fin_items * kTfinSub), dim3(KAON_WG), 0, st, L.descs, L.fin_items, ws, h);
  }
  if (mode == 0 && (mask & (1u << 3))) {
    TclipFn f = gt == KAON_BF16 ? k_tclip<KAON_BF16> : gt == KAON_F16 ? k_tclip<KAON_F16> : k_tclip<KAON_F32>;
    hipLaunchKernelGGL(f, dim3(L.n_tensors), dim3(KAON_WG), 0, st, L.descs, L.n_tensors, ws, h);
  }
  return (int)hipGetLastError();
}

// kaon_momentum_sumsq in torch's order (MSAM norm="tensor").
int torch_momentum_sumsq(const KaonLaunch& L, Ws ws, int codec, hipStream_t st) {
  using Fn = void (*)(const KaonTensor*, int32_t, Ws);
  Fn f = codec == KAON_MOM_F32    ? k_tmsq<KAON_MOM_F32>
         : codec == KAON_MOM_BF16 ? k_tmsq<KAON_MOM_BF16>
         : codec == KAON_MOM_INT8 ? k_tmsq<KAON_MOM_INT8>
         : codec == KAON_MOM_4BIT ? k_tmsq<KAON_MOM_4BIT>
                                  : nullptr;
  if (!f) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(f, dim3(L.n_tensors), dim3(64), 0, st, L.descs, L.n_tensors, ws);
  return (int)hipGetLastError();
}

}  // namespace kaon
