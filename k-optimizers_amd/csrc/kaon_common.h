// kaon_common.h -- workspace views and device helpers shared by the step
// kernels' translation units (kaon_step.hip: phases 1-4, the generic phase-5/6
// kernels, AdaMuon / AdaPNM / KProdigy / MSAM; kaon_fast.hip: the specialized
// phase-5/6 kernels).  Internal to the library.
#pragma once

#include <hip/hip_runtime.h>

#include "kaon_amd.h"
#include "kaon_device.h"

namespace kaon {

// ------------------------------------------------------------ workspace views
struct Ws {
  float* base;
  __device__ KAON_G float* mu(const KaonTensor& T) const { return G(base + T.ws_row); }
  __device__ KAON_G float* rf(const KaonTensor& T) const { return G(base + T.ws_row + T.R); }
  __device__ KAON_G float* rs(const KaonTensor& T) const { return G(base + T.ws_row + 2 * T.R); }
  __device__ KAON_G uint32_t* ramax(const KaonTensor& T) const {
    return G((uint32_t*)(base + T.ws_row + 3 * T.R));
  }
  __device__ KAON_G float* roldsc(const KaonTensor& T) const { return G(base + T.ws_row + 4 * T.R); }
  __device__ KAON_G float* cf(const KaonTensor& T) const { return G(base + T.ws_col); }
  __device__ KAON_G float* part(const KaonTensor& T) const { return G(base + T.ws_part); }
  // the clip's second column partial (t = G^2 / row), laid out as part
  __device__ KAON_G float* part2(const KaonTensor& T) const {
    return G(base + T.ws_part + (int64_t)T.ngroups * T.C);
  }
  __device__ KAON_G uint32_t* bamax(const KaonTensor& T) const { return G((uint32_t*)(base + T.ws_blk)); }
  __device__ KAON_G float* boldsc(const KaonTensor& T, int64_t nb) const { return G(base + T.ws_blk + nb); }
  __device__ KAON_G float* scal(const KaonTensor& T) const { return G(base + T.ws_scal); }
  // generic address of the keep-count word (for atomics)
  __device__ uint32_t* keep_ctr(const KaonTensor& T) const { return (uint32_t*)(base + T.ws_scal) + 1; }
  // AdaMuon: the bf16 momentum, then the orthogonal factor O, [R, C] (first
  // buffer of the Newton-Schulz block)
  __device__ uint16_t* mo(const KaonTensor& T) const { return (uint16_t*)(base + T.ws_aux); }
  // what the row kernels read as "the gradient": O for AdaMuon's factored passes
  __device__ const void* src(const KaonTensor& T, int flags) const {
    return (flags & KAON_F_SRC_O) ? (const void*)mo(T) : T.g;
  }
};

// Streaming accesses: the gradient, parameter and momentum streams of a
// 2.6B-param step are far larger than the caches, so they are loaded and
// stored as non-temporal accesses (NT); small reused arrays (column
// factors, per-row values) are not.
template <bool NT, class V>
__device__ __forceinline__ V ld_stream(const KAON_G V* p) {
  return NT ? __builtin_nontemporal_load(p) : *p;
}
template <class V>
__device__ __forceinline__ void st_stream(KAON_G V* p, V v) {
  __builtin_nontemporal_store(v, p);
}

template <int DT>
__device__ __forceinline__ float round_to(float x) {
  return DT == KAON_BF16 ? rbf(x) : DT == KAON_F16 ? rhf(x) : x;
}
// A 16-bit param / grad of type DT: bits -> fp32, fp32 -> bits (RNE).
template <int DT>
__device__ __forceinline__ float lp2f(uint32_t b) {
  return DT == KAON_F16 ? h2f(b) : bf2f(b);
}
template <int DT>
__device__ __forceinline__ uint32_t f2lp(float f) {
  return DT == KAON_F16 ? f2h(f) : f2bf(f);
}
// Grad-dtype rounding of a GC'd pair (gfx950 conversion for bf16).
template <int GT>
__device__ __forceinline__ void round_pair(float& a, float& b) {
  if (GT == KAON_BF16) {
    rbf2(a, b);
  } else if (GT == KAON_F16) {
    a = rhf(a);
    b = rhf(b);
  }
}

__device__ __forceinline__ int64_t nblocks4(const KaonTensor& T) { return (T.n + T.block4 - 1) / T.block4; }

// Rows [rb, re) of the calling wave inside slice `it` (RW rows per wave).
struct WaveRows {
  int64_t rb, re;
  int w, lane;
};
__device__ __forceinline__ WaveRows wave_rows(const KaonItem& it) {
  WaveRows wr;
  // the wave index is uniform across the wave; readfirstlane tells the compiler
  wr.w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  wr.lane = threadIdx.x & 63;
  const int64_t end = (int64_t)it.row0 + it.nrows;
  wr.rb = min((int64_t)it.row0 + (int64_t)wr.w * it.kind, end);
  wr.re = min(wr.rb + it.kind, end);
  return wr;
}

// Slice sl of a run item (rows [row0 + 4 RW sl, ...), RW = kind) and the
// number of slices in the run.
__device__ __forceinline__ KaonItem slice_item(const KaonItem& run, int sl) {
  KaonItem s = run;
  const int span = 4 * run.kind;
  s.row0 = run.row0 + sl * span;
  s.nrows = min(span, run.nrows - sl * span);
  return s;
}
__device__ __forceinline__ int run_slices(const KaonItem& run) {
  return (run.nrows + 4 * run.kind - 1) / (4 * run.kind);
}
// Column partial of a run: one row of C floats per run.
__device__ __forceinline__ KAON_G float* run_part(const Ws& ws, const KaonTensor& T, const KaonItem& run) {
  return ws.part(T) + (int64_t)(run.row0 / (KAON_RUN * 4 * run.kind)) * T.C;
}

// Chunks of a row: the element range [8c, 8c+8) clipped to the row length.
__device__ __forceinline__ int chunk_cnt(int64_t c, int64_t C) {
  const int64_t j0 = c * 8;
  return j0 >= C ? 0 : (int)min<int64_t>(8, C - j0);
}

// Zero what phase 5 accumulates with atomics (keep-count; 4-bit block absmax
// of blocks that straddle rows).  Run by the phase-1 slice.
__device__ void zero_accumulators(const KaonTensor& T, const KaonItem& it, const Ws& ws, int codec) {
  if (it.row0 == 0 && threadIdx.x == 0) ((KAON_G uint32_t*)ws.scal(T))[1] = 0u;
  if (codec == KAON_MOM_4BIT) {
    const int64_t e_begin = (int64_t)it.row0 * T.C;
    const int64_t e_end = (int64_t)(it.row0 + it.nrows) * T.C;
    if (e_end <= e_begin) return;
    const int64_t b0 = e_begin / T.block4, b1 = (e_end - 1) / T.block4;
    for (int64_t b = b0 + threadIdx.x; b <= b1; b += KAON_WG) ws.bamax(T)[b] = 0u;
  }
}

// The clip's algebraic sum of squares (Adakaon, AdaMuon): the scalar words of
// a tensor hold rm at 4 and the partial sums S_k at 5 + k (one per finalize
// item of KAON_COLITEM columns, or one for a 1-D tensor); phase 4 forms
// ss = rm * (S_0 + S_1 + ...) in item order.
__device__ __forceinline__ int clip_parts(const KaonTensor& T) {
  return T.factored ? (int)((T.C + KAON_COLITEM - 1) / KAON_COLITEM) : 1;
}
__device__ __forceinline__ bool clip_alg(const KaonHyper& hp, int mode) {
  return mode == 0 && hp.clip > 0.0f && !(hp.flags & KAON_F_PNM);
}
// Workgroup sum of one value per thread: the 64-lane xor butterfly per wave,
// then the four wave sums in order (valid in thread 0).  Every thread calls it.
__device__ __forceinline__ float wg_sum4(float a, float* red) {
  const float w = wave_csum(a);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = w;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

// Phase 1 of a 1-D tensor (the whole tensor is one row), by the workgroup:
// v = lerp(v, g*g (+eps1), 1-beta2) (adakaon.py:990-995); AdaPNM:
// v = v*beta2 + (1-beta2)*g*g, mul_ then addcmul_ (one fma in torch), and the
// running max under ams_bound (adapnm.py:1243-1248).  With `scal` (the
// tensor's scalar words) also the clip's sum of (g * g) / v (the new v; no
// eps1) in the algebraic form: thread t adds the elements of chunks t, t+256,
// ... in order, then wg_sum4, into word 5; rm = 1 into word 4.
template <int GT>
__device__ void stats_1d(const KaonTensor& T, const void* gsrc, const KaonHyper& hp, KAON_G float* scal,
                         float* red) {
  const bool clip = scal != nullptr;
  const int64_t C = T.C;
  const int64_t nch = (C + 7) >> 3;
  const bool vec = T.vec_rows != 0;
  const bool eps = (hp.flags & KAON_F_EPS) != 0;
  const bool pnm = (hp.flags & KAON_F_PNM) != 0;
  const bool ams = pnm && (hp.flags & KAON_F_AMS) != 0 && T.max_v;
  float cs = 0.0f;
  for (int64_t c = threadIdx.x; c < nch; c += KAON_WG) {
    const int cnt = chunk_cnt(c, C);
    const bool vv = vec && cnt == 8;
    float x[8], v[8];
    ld8<GT>(gsrc, c * 8, cnt, vv, x);
    ld8<KAON_F32>(T.v, c * 8, cnt, vv, v);
    if (pnm) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = __fmaf_rn(hp.a2 * x[i], x[i], v[i] * hp.b2);
      if (ams) {
        float mx[8];
        ld8<KAON_F32>(T.max_v, c * 8, cnt, vv, mx);
#pragma unroll
        for (int i = 0; i < 8; ++i) mx[i] = fmaxf(mx[i], v[i]);
        st8_f32(T.max_v, c * 8, cnt, vv, mx);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float q = x[i] * x[i];
        if (eps) q = q + hp.eps1;
        v[i] = klerp(v[i], q, hp.w2);
        if (clip && i < cnt) cs = cs + (x[i] * x[i]) / v[i];
      }
    }
    st8_f32(T.v, c * 8, cnt, vv, v);
  }
  if (clip) {
    const float S = wg_sum4(cs, red);
    if (threadIdx.x == 0) {
      scal[4] = 1.0f;
      scal[5] = S;
    }
  }
}

__device__ __forceinline__ void unpack8(const ku4 v, float o[8]) {
  o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xFFFF0000u);
  o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xFFFF0000u);
  o[4] = __uint_as_float(v.z << 16); o[5] = __uint_as_float(v.z & 0xFFFF0000u);
  o[6] = __uint_as_float(v.w << 16); o[7] = __uint_as_float(v.w & 0xFFFF0000u);
}

// Per-row values of a wave group: lane j (< nrows) loads row rb + j's value,
// issued with the chunk loads; lane_val(v, j) hands row j's value to the wave.
__device__ __forceinline__ int64_t lane_row(int64_t rb, int nrows, int lane) {
  return rb + (lane < nrows ? lane : 0);
}
__device__ __forceinline__ float lane_val(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// MSAM perturbation value (msam.py:216-230).  norm="none" (a finite bound b):
// clamp(nan_to_num(x, 0, +b, -b), -b, b); for a bound that is not NaN the clamp
// already takes +-inf to +-b, so only a NaN x needs a case of its own, and it
// becomes 0.  norm="global" / "tensor" (bound +inf): the reference multiplies
// the momentum by its scale with no sanitizing, so x passes as it is and a NaN
// reaches the weights.  `nanfill` is msam_nanfill(bound), formed once per
// launch: 0 for a finite bound, NaN for +inf.
__device__ __forceinline__ float msam_nanfill(float bound) {
  return bound == __builtin_inff() ? __builtin_nanf("") : 0.0f;
}
__device__ __forceinline__ float msam_e(float x, float bound, float nanfill) {
  return x != x ? nanfill : fminf(fmaxf(x, -bound), bound);
}

// Flags of the specialized phase-5/6 kernels: bit 0 GC, 1 cautious, 2 weight
// decay, 3 Nekaon removal, 4 Nekaon climb, 5 the centralized gradient written
// back over p.grad by the apply.
enum { FF_GC = 1, FF_CAUT = 2, FF_WD = 4, FF_NKR = 8, FF_NKC = 16, FF_GCW = 32 };

// Phases 1-4 of an Adakaon step (mode 0) or phase 1 of a Lion step (mode 1)
// with the sums in torch CPU's order (KAON_F_TORCH_ORDER; kaon_torch.hip), for
// the phase bits of `mask`; and kaon_momentum_sumsq's per-tensor sums in that
// order.  Both return a HIP status.
int torch_phases(const KaonLaunch& L, Ws ws, const KaonHyper& h, uint32_t mask, int mode, hipStream_t st);
int torch_momentum_sumsq(const KaonLaunch& L, Ws ws, int codec, hipStream_t st);
// Phase 3 in torch's order (the clip norm's chains) for the tensors of size ranks
// [t0, t1) (descs[k].by_size); a HIP status.
int torch_clip(const KaonLaunch& L, Ws ws, const KaonHyper& h, int32_t t0, int32_t t1, hipStream_t st);

// A phase-5/6 kernel over work items: (descriptors, items, workspace, hyper-parameters).
using ElemFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper);

// The specialized phase-5/6 kernel for (optimizer, phase 5 or 6, codec, FF_*
// flags), or nullptr when none is compiled for that configuration
// (kaon_fast.hip).
ElemFn fast_kernel(int opt, int phase, int codec, int ff);

}  // namespace kaon
