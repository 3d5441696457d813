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
// Work decomposition.  A work item is a slice: 4 wave groups of RW
// consecutive rows of one tensor (RW = max(1, 20 / chunks-per-lane) so a wave
// group spans about 160 elements per lane).  Each wave64 owns its rows whole:
// lane l handles the 8-element chunks l, l+64, ... of every row, so every row
// reduction (GC mean, second-moment row mean, clip sums, int8 absmax) is a
// wave-local butterfly with no LDS or barrier, and per-row values are
// wave-uniform.  The tensor-global dependencies (column factors, row-mean,
// clip divisor, cautious keep-count) split one step into launches:
//   phase 1  slices      GC row means, row EMA, column partials (LDS fold)
//   phase 2  fin items   column EMA + column factors; row mean + row factors
//   phase 3  slices      per-row sums of U^2 (U = G*r*c)
//   phase 4  tensors     clip divisor from the row sums
//   phase 5  slices      cautious keep-count, momentum absmax
//   phase 6  slices      requant + momentum write, cautious rescale, weight
//                        write (SR / RN / kahan / fp32), Nekaon remove+climb
// All reductions follow the CPU oracle's canonical order; there are no
// floating-point atomics, so results are deterministic and bit-exact.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "kaon_common.h"
#include "kaon_device.h"
#include "kaon_ns.h"

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

// Columns per LDS segment of the streamed rows' column fold (phase 1).
constexpr int kSeg = 4096;

// KProdigy's coupled decay folded into the gradient its second moment sees,
// g' = fma(wd, p, GC(g)) (_collect_grad, kprodigy.py:406-414; torch's add with
// alpha is one fused multiply-add), for the generic phase-1 kernel.
__device__ __forceinline__ void add_coupled_wd(const KaonTensor& T, const KaonHyper& hp, int64_t e0, int cnt, bool vv,
                                               float x[8]) {
  float p[8];
  if (hp.p_dtype == KAON_BF16) ld8<KAON_BF16>(T.p, e0, cnt, vv, p);
  else if (hp.p_dtype == KAON_F16) ld8<KAON_F16>(T.p, e0, cnt, vv, p);
  else ld8<KAON_F32>(T.p, e0, cnt, vv, p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = __fmaf_rn(hp.wdl, p[i], x[i]);
}

// =============================================================== phase 1
// The canonical row sum of a row held by an aligned group of 2^lsh <= 32
// lanes (lane cl of the group holding the sum of its chunk cl, 0 past the
// row's chunks).  The 64-lane butterfly of the one-row-per-wave layout adds,
// at offsets 32 ... 2^lsh, only the +0 of lanes past the row, which leaves each
// lane sum x as x + 0 (-0 becomes +0); its offsets 2^(lsh-1) ... 1 pair lanes
// of the same group.  So the sum is that group's butterfly of x + 0.
__device__ __forceinline__ float group_csum(float a, int lsh) {
  float v = a + 0.0f;
  for (int o = (1 << lsh) >> 1; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// Phase 1 of one slice of a factored tensor whose rows have at most 32 chunks
// (the register layouts, RW > 1 rows per wave group, no coupled decay).  A
// wave works on 64 / L of its rows side by side, L = 2^ceil(log2(chunks))
// lanes per row, lane cl of a row's group taking chunk cl: one memory round
// trip per 64 / L rows instead of one per row.  Every value and every sum
// order is that of k_stats's one-row-at-a-time body: the row sums through
// group_csum, and each column partial (the wave group's rows added in row
// order, then the wave groups folded in order in LDS) built by lane group 0,
// which takes each row's values from that row's lane group in turn.
template <int GT>
__device__ __forceinline__ void stats_packed(const KaonTensor& T, const KaonItem& sit, const Ws& ws,
                                             const KaonHyper& hp, int mode, const void* gsrc, KAON_G float* part,
                                             KAON_G float* part2, bool first, bool alg, float* lds_col) {
  const int64_t C = T.C;
  const int nch = (int)((C + 7) >> 3);
  const bool vec = T.vec_rows != 0;
  const bool eps = (hp.flags & KAON_F_EPS) != 0;
  const bool gc = (hp.flags & KAON_F_GC) != 0;
  const WaveRows wr = wave_rows(sit);
  const int lsh = nch <= 1 ? 0 : 32 - __builtin_clz((uint32_t)(nch - 1));
  const int P = 64 >> lsh;
  const int grp = wr.lane >> lsh;
  const int cl = wr.lane & ((1 << lsh) - 1);
  const int cnt0 = chunk_cnt(cl, C);  // elements of the lane's chunk in any row
  KAON_G float* mu_arr = ws.mu(T);
  float colacc[8], acc2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    colacc[i] = 0.0f;
    acc2[i] = 0.0f;
  }
  for (int64_t r0 = wr.rb; r0 < wr.re; r0 += P) {
    const int nv = (int)min<int64_t>(P, wr.re - r0);  // rows of this pass (wave-uniform)
    const bool rvalid = grp < nv;
    const int64_t r = rvalid ? r0 + grp : wr.rb;
    const int cnt = rvalid ? cnt0 : 0;
    float x[8];
    if (cnt > 0) {
      ld8<GT>(gsrc, r * C + (int64_t)cl * 8, cnt, vec && cnt == 8, x);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = 0.0f;
    }
    const float row_old = mode == 0 ? T.row[r] : 0.0f;
    float xb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xb[i] = x[i];
    float mu = 0.0f;
    if (gc) {
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < cnt) a = a + x[i];
      mu = round_to<GT>(group_csum(a, lsh) / (float)C);
      if (rvalid && cl == 0) mu_arr[r] = mu;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float a0 = xb[i] - mu, a1 = xb[i + 1] - mu;
        round_pair<GT>(a0, a1);
        xb[i] = a0;
        xb[i + 1] = a1;
      }
    }
    if (mode == 1) continue;
    float q[8];
    float a2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      q[i] = xb[i] * xb[i];
      if (eps) q[i] = q[i] + hp.eps1;
      if (i < cnt) a2 = a2 + q[i];
    }
    const float s2 = group_csum(a2, lsh);
    const float nr = klerp(row_old, s2 / (float)C, hp.w2);
    if (rvalid && cl == 0) T.row[r] = nr;
    // the column partial: rows r0, r0 + 1, ... in order
    for (int g = 0; g < nv; ++g) {
      const int src = (g << lsh) + cl;
#pragma unroll
      for (int i = 0; i < 8; ++i) colacc[i] = colacc[i] + __shfl(q[i], src, 64);
    }
    if (alg) {
      // the clip's second column partial, t = (G * G) / row (the new row; no
      // eps1), G formed again from the raw gradient as the row-by-row body does
      const float w = 1.0f / nr;
      float t[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float gv = gc ? round_to<GT>(x[i] - mu) : x[i];
        t[i] = (gv * gv) * w;
      }
      for (int g = 0; g < nv; ++g) {
        const int src = (g << lsh) + cl;
        const bool start = r0 == wr.rb && g == 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float tv = __shfl(t[i], src, 64);
          acc2[i] = start ? tv : acc2[i] + tv;
        }
      }
    }
  }
  if (mode == 1) return;
  // fold the wave-group partials in group order into the slice partial (lane
  // group 0 holds them, lane cl for chunk cl), then into the run partial
  const bool has_rows = wr.re > wr.rb;
  const bool holder = grp == 0 && has_rows;
  for (int wf = 0; wf < 4; ++wf) {
    if (wr.w == wf && holder) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < cnt0) {
          const int j = cl * 8 + i;
          lds_col[j] = wf == 0 ? colacc[i] : lds_col[j] + colacc[i];
        }
    }
    __syncthreads();
  }
  for (int64_t j = threadIdx.x; j < C; j += KAON_WG) part[j] = first ? lds_col[j] : part[j] + lds_col[j];
  __syncthreads();  // lds_col is reused
  if (!alg) return;
  for (int wf = 0; wf < 4; ++wf) {
    if (wr.w == wf && holder) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < cnt0) {
          const int j = cl * 8 + i;
          lds_col[j] = wf == 0 ? acc2[i] : lds_col[j] + acc2[i];
        }
    }
    __syncthreads();
  }
  for (int64_t j = threadIdx.x; j < C; j += KAON_WG) part2[j] = first ? lds_col[j] : part2[j] + lds_col[j];
  __syncthreads();  // lds_col is reused by the next slice
}

// mode 0 (Adakaon): GC row mean (stored), row EMA of mean_C(G^2), column
// partial of the slice (wave groups folded in order in LDS); 1-D tensors: v
// EMA.  mode 1 (Lion): GC row means only.  CPL > 0 keeps a row of up to CPL
// chunks per lane in registers; CPL == 0 streams the row from memory (used for
// rows longer than 24 chunks per lane, fp32 grads with long rows, and 1-D).
// With KAON_F_PD_COUPLED (KProdigy, factored, coupled decay) G is the decayed
// gradient fma(wd, p, GC(g)); the GC mean is still the raw gradient's.
template <int GT, int CPL>
__global__ __launch_bounds__(KAON_WG) void k_stats(const KaonTensor* __restrict__ D,
                                                   const KaonItem* __restrict__ items, Ws ws, KaonHyper hp,
                                                   int mode) {
  extern __shared__ float lds_col[];
  __shared__ float winv_s[4][KAON_ROW_BUDGET];  // 1 / row (the new row) of each wave's rows
  __shared__ float red4[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  // KProdigy's per-element v and its block-factored tensors: their own pass 1 kernels
  if (T.full_v || T.fb_r) return;
  zero_accumulators(T, it, ws, hp.codec);
  const void* gsrc = ws.src(T, hp.flags);
  const int64_t C = T.C;
  const int64_t nch = (C + 7) >> 3;
  const int cpl = (int)((nch + 63) >> 6);
  const bool vec = T.vec_rows != 0;
  const bool eps = (hp.flags & KAON_F_EPS) != 0;
  const bool alg = clip_alg(hp, mode);
  const bool cwd = mode == 0 && (hp.flags & KAON_F_PD_COUPLED) != 0;

  if (!T.factored) {
    if (mode == 0) stats_1d<GT>(T, gsrc, hp, alg ? ws.scal(T) : nullptr, red4);
    return;
  }

  const bool gc = (hp.flags & KAON_F_GC) != 0;
  if (mode == 1 && !gc) return;
  KAON_G float* mu_arr = ws.mu(T);
  const int RW = it.kind;
  KAON_G float* part = run_part(ws, T, it);
  const int nsl = run_slices(it);
  // rows of at most 32 chunks (the class of 1-4 chunks per lane): side by side
  const bool packed = CPL == 4 && nch <= 32 && RW > 1 && !cwd;
#pragma clang loop unroll(disable)
  for (int sl = 0; sl < nsl; ++sl) {
  if constexpr (CPL == 4) {
    if (packed) {
      stats_packed<GT>(T, slice_item(it, sl), ws, hp, mode, gsrc, part, part + (int64_t)T.ngroups * C, sl == 0, alg,
                       lds_col);
      continue;
    }
  }
  const WaveRows wr = wave_rows(slice_item(it, sl));

  // registers: row buffer (CPL chunks) and the wave-group column partial
  constexpr int NB = CPL > 0 ? CPL : 1;
  float xb[NB][8];
  float colacc[NB][8];
#pragma unroll
  for (int k = 0; k < NB; ++k)
#pragma unroll
    for (int i = 0; i < 8; ++i) colacc[k][i] = 0.0f;

  for (int64_t r = wr.rb; r < wr.re; ++r) {
    const int64_t rowoff = r * C;
    float mu = 0.0f;
    if (CPL > 0) {
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const int64_t c = wr.lane + 64 * k;
        const int cnt = k < cpl ? chunk_cnt(c, C) : 0;
        if (cnt > 0) ld8<GT>(gsrc, rowoff + c * 8, cnt, vec && cnt == 8, xb[k]);
        else
#pragma unroll
          for (int i = 0; i < 8; ++i) xb[k][i] = 0.0f;
      }
      if (gc) {
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
          const int cnt = k < cpl ? chunk_cnt(wr.lane + 64 * k, C) : 0;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i < cnt) a = a + xb[k][i];
        }
        mu = round_to<GT>(wave_csum(a) / (float)C);
        if (wr.lane == 0) mu_arr[r] = mu;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            float a0 = xb[k][i] - mu, a1 = xb[k][i + 1] - mu;
            round_pair<GT>(a0, a1);
            xb[k][i] = a0;
            xb[k][i + 1] = a1;
          }
        }
      }
      if (mode == 1) continue;
      if (cwd) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
          const int64_t c = wr.lane + 64 * k;
          const int cnt = k < cpl ? chunk_cnt(c, C) : 0;
          if (cnt > 0) add_coupled_wd(T, hp, rowoff + c * 8, cnt, vec && cnt == 8, xb[k]);
        }
      }
      float a2 = 0.0f;
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const int cnt = k < cpl ? chunk_cnt(wr.lane + 64 * k, C) : 0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i < cnt) {
            float q = xb[k][i] * xb[k][i];
            if (eps) q = q + hp.eps1;
            a2 = a2 + q;
            if (RW > 1) colacc[k][i] = colacc[k][i] + q;
          }
      }
      const float s2 = wave_csum(a2);
      const float nr = klerp(T.row[r], s2 / (float)C, hp.w2);
      if (wr.lane == 0) {
        T.row[r] = nr;
        if (alg) winv_s[wr.w][r - wr.rb] = 1.0f / nr;
      }
    } else {
      // streaming: sweep A (GC sum), sweep B (q and the row sum)
      if (gc) {
        float a = 0.0f;
        for (int k = 0; k < cpl; ++k) {
          const int64_t c = wr.lane + 64 * k;
          const int cnt = chunk_cnt(c, C);
          if (cnt <= 0) continue;
          float x[8];
          ld8<GT>(gsrc, rowoff + c * 8, cnt, vec && cnt == 8, x);
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i < cnt) a = a + x[i];
        }
        mu = round_to<GT>(wave_csum(a) / (float)C);
        if (wr.lane == 0) mu_arr[r] = mu;
      }
      if (mode == 1) continue;
      float a2 = 0.0f;
      for (int k = 0; k < cpl; ++k) {
        const int64_t c = wr.lane + 64 * k;
        const int cnt = chunk_cnt(c, C);
        if (cnt <= 0) continue;
        float x[8];
        ld8<GT>(gsrc, rowoff + c * 8, cnt, vec && cnt == 8, x);
        if (gc) {
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = round_to<GT>(x[i] - mu);
        }
        if (cwd) add_coupled_wd(T, hp, rowoff + c * 8, cnt, vec && cnt == 8, x);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i < cnt) {
            float q = x[i] * x[i];
            if (eps) q = q + hp.eps1;
            a2 = a2 + q;
          }
      }
      const float s2 = wave_csum(a2);
      const float nr = klerp(T.row[r], s2 / (float)C, hp.w2);
      if (wr.lane == 0) {
        T.row[r] = nr;
        if (alg) winv_s[wr.w][r - wr.rb] = 1.0f / nr;
      }
    }
  }
  if (mode == 1) continue;

  // fold the wave-group partials in group order into the slice partial
  const bool has_rows = wr.re > wr.rb;
  if (CPL == 0) {
    // streamed rows (RW == 1, any length): the slice partial is folded kSeg
    // columns at a time through LDS.  Per column the order is the one below:
    // wave 0 + wave 1 + wave 2 + wave 3, then the slice added to the run partial.
    for (int64_t c0 = 0; c0 < C; c0 += kSeg) {
      const int64_t c1 = min(C, c0 + (int64_t)kSeg);
      for (int wf = 0; wf < 4; ++wf) {
        if (wr.w == wf && has_rows) {
          const int64_t r = wr.rb;
          const float mu = gc ? mu_arr[r] : 0.0f;
          for (int64_t c = (c0 >> 3) + wr.lane; c * 8 < c1; c += 64) {
            const int cnt = chunk_cnt(c, C);
            float x[8];
            ld8<GT>(gsrc, r * C + c * 8, cnt, vec && cnt == 8, x);
            if (gc) {
#pragma unroll
              for (int i = 0; i < 8; ++i) x[i] = round_to<GT>(x[i] - mu);
            }
            if (cwd) add_coupled_wd(T, hp, r * C + c * 8, cnt, vec && cnt == 8, x);
#pragma unroll
            for (int i = 0; i < 8; ++i)
              if (i < cnt) {
                float v = x[i] * x[i];
                if (eps) v = v + hp.eps1;
                const int64_t j = c * 8 + i - c0;
                lds_col[j] = wf == 0 ? v : lds_col[j] + v;
              }
          }
        }
        __syncthreads();
      }
      for (int64_t j = c0 + threadIdx.x; j < c1; j += KAON_WG)
        part[j] = sl == 0 ? lds_col[j - c0] : part[j] + lds_col[j - c0];
      __syncthreads();  // lds_col is reused by the next segment
    }
  } else {
  for (int wf = 0; wf < 4; ++wf) {
    if (wr.w == wf && has_rows) {
      if (CPL > 0) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
          const int64_t c = wr.lane + 64 * k;
          const int cnt = k < cpl ? chunk_cnt(c, C) : 0;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i < cnt) {
              float v;
              if (RW > 1) {
                v = colacc[k][i];
              } else {
                v = xb[k][i] * xb[k][i];
                if (eps) v = v + hp.eps1;
              }
              const int64_t j = c * 8 + i;
              lds_col[j] = wf == 0 ? v : lds_col[j] + v;
            }
        }
      }
    }
    __syncthreads();
  }
  // the run partial: the slice partials added in slice order
  for (int64_t j = threadIdx.x; j < C; j += KAON_WG) part[j] = sl == 0 ? lds_col[j] : part[j] + lds_col[j];
  __syncthreads();  // lds_col is reused by the next slice
  }
  if (!alg) continue;
  // The clip's second column partial, t = (G * G) / row (the new row; no
  // eps1), in the same wave-group / slice / run order, the rows read again
  // (this kernel serves the grad layouts outside the prefetching kernels'
  // register budget).
  KAON_G float* part2 = part + (int64_t)T.ngroups * C;
  const int64_t segC = CPL > 0 ? C : (int64_t)kSeg;
  for (int64_t c0 = 0; c0 < C; c0 += segC) {
    const int64_t c1 = min(C, c0 + segC);
    for (int wf = 0; wf < 4; ++wf) {
      if (wr.w == wf && has_rows) {
        for (int64_t c = (c0 >> 3) + wr.lane; c * 8 < c1; c += 64) {
          const int cnt = chunk_cnt(c, C);
          float acc[8];
          for (int64_t r = wr.rb; r < wr.re; ++r) {
            const float mu = gc ? mu_arr[r] : 0.0f;
            const float w = winv_s[wf][r - wr.rb];
            float x[8];
            ld8<GT>(gsrc, r * C + c * 8, cnt, vec && cnt == 8, x);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float gv = gc ? round_to<GT>(x[i] - mu) : x[i];
              const float t = (gv * gv) * w;
              acc[i] = r == wr.rb ? t : acc[i] + t;
            }
          }
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i < cnt) {
              const int64_t j = c * 8 + i - c0;
              lds_col[j] = wf == 0 ? acc[i] : lds_col[j] + acc[i];
            }
        }
      }
      __syncthreads();
    }
    for (int64_t j = c0 + threadIdx.x; j < c1; j += KAON_WG)
      part2[j] = sl == 0 ? lds_col[j - c0] : part2[j] + lds_col[j - c0];
    __syncthreads();  // lds_col is reused by the next segment or slice
  }
  }
}

// =============================================================== phase 2
// Finalize items.  kind 0: col = lerp(col, colsum/R, 1-beta2), cf = 1/sqrt(col)
// for columns [row0, row0+nrows), colsum = the run partials added in run
// order; with the algebraic clip sum also the item's partial S_k = sum of
// colsum2_j / col_j (thread t adds columns t, t+256, ... in order, then
// wg_sum4).  kind 1: rm = mean(row) (canonical sum), rf = 1/sqrt(row/rm)
// (_factored.py:48-52, 76-82); rm is kept in the tensor's scalar word 4.
__device__ __forceinline__ float run_sum(const KAON_G float* part, int ngroups, int64_t C, int64_t j) {
  float cs = 0.0f;
  int g = 0;
  for (; g + 8 <= ngroups; g += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(g + u) * C + j];
#pragma unroll
    for (int u = 0; u < 8; ++u) cs = cs + v[u];
  }
  for (; g < ngroups; ++g) cs = cs + part[(int64_t)g * C + j];
  return cs;
}
__global__ __launch_bounds__(KAON_WG) void k_fin(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ float rm_s;
  __shared__ float red4[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t R = T.R, C = T.C;
  if (it.kind == 0) {
    const bool alg = clip_alg(hp, 0);
    const KAON_G float* part = ws.part(T);
    const KAON_G float* part2 = ws.part2(T);
    KAON_G float* cf = ws.cf(T);
    float a = 0.0f;
    for (int64_t j = it.row0 + threadIdx.x; j < (int64_t)it.row0 + it.nrows; j += KAON_WG) {
      const float cs = run_sum(part, T.ngroups, C, j);
      const float nc = klerp(T.col[j], cs / (float)R, hp.w2);
      T.col[j] = nc;
      cf[j] = 1.0f / sqrtf(nc);
      if (alg) a = a + run_sum(part2, T.ngroups, C, j) / nc;
    }
    if (alg) {
      const float S = wg_sum4(a, red4);
      if (threadIdx.x == 0) ws.scal(T)[5 + it.row0 / KAON_COLITEM] = S;
    }
  } else {
    if (threadIdx.x < 64) {
      const int64_t nch = (R + 7) >> 3;
      float a = 0.0f;
      for (int64_t c = threadIdx.x; c < nch; c += 64)
        for (int i = 0; i < 8; ++i) {
          const int64_t j = c * 8 + i;
          if (j < R) a = a + T.row[j];
        }
      const float s = wave_csum(a);
      if (threadIdx.x == 0) {
        rm_s = s / (float)R;
        ws.scal(T)[4] = s / (float)R;
      }
    }
    __syncthreads();
    const float rm = rm_s;
    KAON_G float* rf = ws.rf(T);
    for (int64_t i = threadIdx.x; i < R; i += KAON_WG) rf[i] = 1.0f / sqrtf(T.row[i] / rm);
  }
}

// =============================================================== phase 4
// Clip divisor of every tensor: max(RMS(U) / clip, 1), RMS(U) = sqrt(ss) /
// sqrt(n) (_factored.py:84-89 via adakaon.py:1001-1003).  Adakaon and AdaMuon
// take ss in the algebraic form rm * (S_0 + S_1 + ...) (the item partials in
// item order, from phases 1-2); AdaPNM as the canonical sum over the row sums
// rs of U^2 of its phase 3.  One wave per tensor.
__global__ __launch_bounds__(KAON_WG) void k_clipdiv(const KaonTensor* __restrict__ D, int32_t n_tensors, Ws ws,
                                                     KaonHyper hp) {
  const int t = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (t >= n_tensors) return;
  const KaonTensor& T = D[t];
  if (T.n == 0) return;
  const int lane = threadIdx.x & 63;
  const int64_t R = T.R;
  float ss;
  if (clip_alg(hp, 0)) {
    const KAON_G float* sc = ws.scal(T);
    const int np = clip_parts(T);
    float S = 0.0f;
    for (int k = 0; k < np; ++k) S = S + sc[5 + k];
    ss = sc[4] * S;
  } else {
    const KAON_G float* rs = ws.rs(T);
    float a = 0.0f;
    for (int64_t c = lane; c * 8 < R; c += 64) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = rs[min(c * 8 + i, R - 1)];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c * 8 + i < R) a = a + v[i];
    }
    ss = wave_csum(a);
  }
  // clip_threshold 0 (AdaPNM) leaves the update unclipped (adapnm.py:157-161)
  if (lane == 0) ws.scal(T)[0] = hp.clip > 0.0f ? fmaxf((sqrtf(ss) / T.sqrt_n) / hp.clip, 1.0f) : 1.0f;
}

// =============================================================== prefetching row kernels
// Phase 1 for slices of bf16 grads with 16-byte rows (C % 8 == 0) of at
// most 24 chunks per lane.  A wave loads its whole wave group (RW rows, RW *
// CPL <= 24 chunks per lane) into registers as packed bf16 with every load
// issued before the first use, so each lane keeps up to 24 x 16 bytes in
// flight; the row reductions and the column fold then run from registers.
// The arithmetic and its order are those of k_stats.

// Chunk k of the lane in each of the wave group's rows.  Every load is
// issued unconditionally from a valid address (rows past the group and
// chunks past the row end load the last ones again, and a wave without rows
// loads row `rsafe`), so no load waits behind a divergent branch; the caller
// ignores the extra values.
template <int CPL, int RW>
__device__ __forceinline__ void load_group(const uint16_t* __restrict__ g, int64_t rb, int nrows, int64_t rsafe,
                                           int64_t C, int nch, int lane, ku4 (&raw)[RW][CPL]) {
  uint32_t off[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) off[k] = 16u * (uint32_t)min(lane + 64 * k, nch - 1);
#pragma unroll
  for (int j = 0; j < RW; ++j) {
    const int64_t r = nrows > 0 ? rb + min(j, nrows - 1) : rsafe;
    const KAON_G uint8_t* rowp = (const KAON_G uint8_t*)G(g + r * C);
#pragma unroll
    for (int k = 0; k < CPL; ++k) raw[j][k] = ld_stream<true>((const KAON_G ku4*)(rowp + off[k]));
  }
}

// q = (G - mu)^2 (+ eps1) of one chunk, G - mu rounded to bf16 (GC in the
// grad dtype).  EPS 0: no eps1; 2: x*x + eps1 rounded twice; 1: the same as
// one fused multiply-add, which gives the same bits for every bf16-valued x
// when eps1 is 0 or at least 2^-100: x*x is exact unless |x| < 2^-67, and
// then x*x < 2^-134 lies below half an ulp of eps1, so both forms give eps1.
// With gc the chunk's GC'd values replace it in `v` (bf16 pairs packed as
// loaded), for the clip partial's second pass over the row registers.
template <int EPS>
__device__ __forceinline__ void sq_chunk(ku4& v, float mu, bool gc, float e1, float q[8]) {
  float x[8];
  if (gc) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a0 = __uint_as_float(w[i] << 16) - mu, a1 = __uint_as_float(w[i] & 0xFFFF0000u) - mu;
      w[i] = f2bf2(a0, a1);
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
    v = ku4{w[0], w[1], w[2], w[3]};
  } else {
    unpack8(v, x);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = EPS == 1 ? __fmaf_rn(x[i], x[i], e1) : EPS == 2 ? x[i] * x[i] + e1 : x[i] * x[i];
}
// q of a chunk whose values are final (GC'd in place by sq_chunk).
template <int EPS>
__device__ __forceinline__ void sq_plain(const ku4 v, float e1, float q[8]) {
  float x[8];
  unpack8(v, x);
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = EPS == 1 ? __fmaf_rn(x[i], x[i], e1) : EPS == 2 ? x[i] * x[i] + e1 : x[i] * x[i];
}

// Column partial of a slice, segment by segment: segment k is chunk k of
// every lane (columns 512k .. 512k+511).  Each wave writes its wave group's
// partial for the segment into its LDS slot, and after one barrier every
// thread forms the ordered sum ((w0 + w1) + w2) + w3 of two columns and
// stores it (two LDS buffers alternate, so one barrier per segment suffices).
__device__ __forceinline__ void seg_put(float (*seg)[512], int w, int lane, const float v[8]) {
  kf4* d = (kf4*)(&seg[w][lane * 8]);
  d[0] = kf4{v[0], v[1], v[2], v[3]};
  d[1] = kf4{v[4], v[5], v[6], v[7]};
}
// The run partial (the slice partials added in slice order) is kept in
// `racc` (LDS, C floats; each thread owns its two columns) and stored to
// `part` after the last slice, or, with racc == nullptr, accumulated in
// `part` itself.
__device__ __forceinline__ void seg_fold(float (*seg)[512], int nw, int64_t col0, int64_t C, KAON_G float* part,
                                         bool acc, bool last, int tid, float* racc) {
  const int c = 2 * tid;
  if (col0 + c >= C) return;  // C % 8 == 0: both columns are in range or neither
  float a0 = seg[0][c], a1 = seg[0][c + 1];
  for (int w = 1; w < nw; ++w) {
    a0 = a0 + seg[w][c];
    a1 = a1 + seg[w][c + 1];
  }
  KAON_G ku2* dst = (KAON_G ku2*)(part + col0 + c);
  if (racc) {
    float* r = racc + col0 + c;
    if (acc) {
      a0 = r[0] + a0;
      a1 = r[1] + a1;
    }
    if (!last) {
      r[0] = a0;
      r[1] = a1;
      return;
    }
  } else if (acc) {
    const ku2 o = *dst;
    a0 = __uint_as_float(o.x) + a0;
    a1 = __uint_as_float(o.y) + a1;
  }
  *dst = ku2{__float_as_uint(a0), __float_as_uint(a1)};
}
// seg_fold with the run partial of the thread's two columns of segment k in
// registers (r0, r1) instead of LDS; the order is the same.
__device__ __forceinline__ void seg_fold_reg(float (*seg)[512], int nw, int64_t col0, int64_t C,
                                             KAON_G float* part, bool acc, bool last, int tid, float& r0,
                                             float& r1) {
  const int c = 2 * tid;
  if (col0 + c >= C) return;
  float a0 = seg[0][c], a1 = seg[0][c + 1];
  for (int w = 1; w < nw; ++w) {
    a0 = a0 + seg[w][c];
    a1 = a1 + seg[w][c + 1];
  }
  if (acc) {
    a0 = r0 + a0;
    a1 = r1 + a1;
  }
  if (!last) {
    r0 = a0;
    r1 = a1;
    return;
  }
  *(KAON_G ku2*)(part + col0 + c) = ku2{__float_as_uint(a0), __float_as_uint(a1)};
}

// The second (clip) partial's run accumulator: racc2 in LDS (REG2 false), or
// the thread's two columns per segment in registers rr2 (REG2 true).
template <int CPL, int RW, int EPS, bool REG2>
__device__ __forceinline__ void pf_stats_body(const KaonTensor& T, const KaonItem& it, const Ws& ws,
                                              const KaonHyper& hp, int mode, float (*seg)[4][512],
                                              KAON_G float* part, bool acc, bool last, float* racc,
                                              KAON_G float* part2, float* racc2, float (&rr2)[48]) {
  const int64_t C = T.C;
  const int nch = (int)(C >> 3);
  WaveRows wr = wave_rows(it);
  // recomputed per slice: values derived from the lane are not kept live
  // across the slice loop
  asm volatile("" : "+v"(wr.lane));
  int tid = (int)threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int nrows = (int)(wr.re - wr.rb);
  const bool gc = (hp.flags & KAON_F_GC) != 0;
  const float e1 = hp.eps1;
  if (mode == 1 && (!gc || nrows <= 0)) return;
  const int64_t rl = lane_row(wr.rb, nrows, wr.lane);
  const float row_old = (mode == 0 && nrows > 0) ? G(T.row)[rl] : 0.0f;
  const void* gsrc = ws.src(T, hp.flags);
  ku4 raw[RW][CPL];
  load_group<CPL, RW>((const uint16_t*)gsrc, wr.rb, nrows, it.row0, C, nch, wr.lane, raw);
  // GC means of the wave's rows; both per-row divisions by C are exact
  // through the fp64 reciprocal (div_r64)
  const double rc = rcp64((float)C);
  float mu[RW];
  KAON_G float* mu_arr = ws.mu(T);
#pragma unroll
  for (int j = 0; j < RW; ++j) {
    mu[j] = 0.0f;
    if (j >= nrows || !gc) continue;
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      if (wr.lane + 64 * k < nch) {
        float x[8];
        unpack8(raw[j][k], x);
#pragma unroll
        for (int i = 0; i < 8; ++i) a = a + x[i];
      }
    }
    mu[j] = rbf(div_r64(wave_csum(a), rc));
    if (wr.lane == 0) mu_arr[wr.rb + j] = mu[j];
  }
  if (mode == 1) return;
  // q = (G - mu)^2 (+eps1) once per element: into the row sums (lane order:
  // chunk by chunk) and the wave group's column partial (row order)
  const int nw = (int)min<int64_t>(4, ((int64_t)it.nrows + RW - 1) / RW);
  // Segments per barrier: the wide class (REG2: the clip's run partial in
  // registers) has the LDS for two, so it waits half as often.  The buffer
  // sets alternate from one barrier group to the next, across both passes;
  // each column's partials are added in the same order either way.
  constexpr int SEGG = REG2 ? 2 : 1;
  constexpr int NG = (CPL + SEGG - 1) / SEGG;  // barrier groups per pass
  auto sbuf = [&](int pass, int k) { return seg[((pass * NG + k / SEGG) & 1) * SEGG + k % SEGG]; };
  float a2[RW];
#pragma unroll
  for (int j = 0; j < RW; ++j) a2[j] = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    if (nrows > 0) {
      float v[8];
      const bool in = wr.lane + 64 * k < nch;
#pragma unroll
      for (int j = 0; j < RW; ++j) {
        if (j < nrows) {
          float q[8];
          sq_chunk<EPS>(raw[j][k], mu[j], gc, e1, q);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (in) a2[j] = a2[j] + q[i];
            v[i] = j == 0 ? q[i] : v[i] + q[i];
          }
        }
      }
      seg_put(sbuf(0, k), wr.w, wr.lane, v);
    }
    if (k % SEGG == SEGG - 1 || k == CPL - 1) {
      __syncthreads();
#pragma unroll
      for (int kk = k - k % SEGG; kk <= k; ++kk)
        seg_fold(sbuf(0, kk), nw, (int64_t)kk * 512, C, part, acc, last, tid, racc);
    }
  }
  float wr_inv[RW];  // 1 / row_j (the new row) for the clip partial
#pragma unroll
  for (int j = 0; j < RW; ++j) {
    wr_inv[j] = 0.0f;
    if (j >= nrows) continue;
    const float s2 = wave_csum(a2[j]);
    const float rv = lane_val(row_old, j);
    const float nr = klerp(rv, div_r64(s2, rc), hp.w2);
    if (wr.lane == 0) G(T.row)[wr.rb + j] = nr;
    wr_inv[j] = 1.0f / nr;
  }
  if (!clip_alg(hp, mode)) return;
  // The clip's second column partial, t = (G * G) / row (no eps1: rows of
  // zeros add nothing), from the registers (GC'd in place by the first pass),
  // in the same wave-group / slice / run order.  The LDS segment buffers keep
  // alternating from the first pass's.
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    if (nrows > 0) {
      float v[8];
#pragma unroll
      for (int j = 0; j < RW; ++j) {
        if (j < nrows) {
          float q[8];
          sq_plain<0>(raw[j][k], e1, q);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float t = q[i] * wr_inv[j];
            v[i] = j == 0 ? t : v[i] + t;
          }
        }
      }
      seg_put(sbuf(1, k), wr.w, wr.lane, v);
    }
    if (k % SEGG == SEGG - 1 || k == CPL - 1) {
      __syncthreads();
#pragma unroll
      for (int kk = k - k % SEGG; kk <= k; ++kk) {
        if (REG2)
          seg_fold_reg(sbuf(1, kk), nw, (int64_t)kk * 512, C, part2, acc, last, tid, rr2[2 * kk], rr2[2 * kk + 1]);
        else
          seg_fold(sbuf(1, kk), nw, (int64_t)kk * 512, C, part2, acc, last, tid, racc2);
      }
    }
  }
}

// Row class 0: 1-4 chunks per lane, 1 class 1: 5-10, class 2: 11-24; the
// body is specialized on the exact chunks per lane and its rows per wave
// group (RW = max(1, KAON_ROW_BUDGET / CPL)).
#define KAON_COMMA ,
#define KAON_PF_SWITCH(CLS, BODY, X, ...)                                                      \
  switch (cpl) {                                                                                \
    case 1: if (CLS == 0) BODY<1, 20 X>(__VA_ARGS__); break;                                   \
    case 2: if (CLS == 0) BODY<2, 10 X>(__VA_ARGS__); break;                                   \
    case 3: if (CLS == 0) BODY<3, 6 X>(__VA_ARGS__); break;                                    \
    case 4: if (CLS == 0) BODY<4, 5 X>(__VA_ARGS__); break;                                    \
    case 5: if (CLS == 1) BODY<5, 4 X>(__VA_ARGS__); break;                                    \
    case 6: if (CLS == 1) BODY<6, 3 X>(__VA_ARGS__); break;                                    \
    case 7: if (CLS == 1) BODY<7, 2 X>(__VA_ARGS__); break;                                    \
    case 8: if (CLS == 1) BODY<8, 2 X>(__VA_ARGS__); break;                                    \
    case 9: if (CLS == 1) BODY<9, 2 X>(__VA_ARGS__); break;                                    \
    case 10: if (CLS == 1) BODY<10, 2 X>(__VA_ARGS__); break;                                  \
    case 11: if (CLS == 2) BODY<11, 1 X>(__VA_ARGS__); break;                                  \
    case 12: if (CLS == 2) BODY<12, 1 X>(__VA_ARGS__); break;                                  \
    case 13: if (CLS == 2) BODY<13, 1 X>(__VA_ARGS__); break;                                  \
    case 14: if (CLS == 2) BODY<14, 1 X>(__VA_ARGS__); break;                                  \
    case 15: if (CLS == 2) BODY<15, 1 X>(__VA_ARGS__); break;                                  \
    case 16: if (CLS == 2) BODY<16, 1 X>(__VA_ARGS__); break;                                  \
    case 17: if (CLS == 2) BODY<17, 1 X>(__VA_ARGS__); break;                                  \
    case 18: if (CLS == 2) BODY<18, 1 X>(__VA_ARGS__); break;                                  \
    case 19: if (CLS == 2) BODY<19, 1 X>(__VA_ARGS__); break;                                  \
    case 20: if (CLS == 2) BODY<20, 1 X>(__VA_ARGS__); break;                                  \
    case 21: if (CLS == 2) BODY<21, 1 X>(__VA_ARGS__); break;                                  \
    case 22: if (CLS == 2) BODY<22, 1 X>(__VA_ARGS__); break;                                  \
    case 23: if (CLS == 2) BODY<23, 1 X>(__VA_ARGS__); break;                                  \
    case 24: if (CLS == 2) BODY<24, 1 X>(__VA_ARGS__); break;                                  \
  }

template <int CLS, int EPS, bool REG2>
__device__ __forceinline__ void pf_stats_run(const KaonTensor* __restrict__ D, const KaonItem* __restrict__ items,
                                             const Ws& ws, const KaonHyper& hp, int mode, float (*seg)[4][512],
                                             float* racc, float* racc2) {
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  // KProdigy's per-element v and its block-factored tensors: their own pass 1 kernels
  if (T.full_v || T.fb_r) return;
  zero_accumulators(T, it, ws, hp.codec);
  const int cpl = (int)(((T.C >> 3) + 63) >> 6);
  KAON_G float* part = run_part(ws, T, it);
  KAON_G float* part2 = part + (int64_t)T.ngroups * T.C;
  const int nsl = run_slices(it);
  float rr2[48];
#pragma unroll
  for (int i = 0; i < 48; ++i) rr2[i] = 0.0f;
#pragma clang loop unroll(disable)
  for (int sl = 0; sl < nsl; ++sl) {
    if (sl > 0) __syncthreads();  // the LDS fold buffers are reused
    const KaonItem si = slice_item(it, sl);
    KAON_PF_SWITCH(CLS, pf_stats_body, KAON_COMMA EPS KAON_COMMA REG2, T, si, ws, hp, mode, seg, part, sl > 0,
                   sl + 1 == nsl, racc, part2, racc2, rr2)
  }
}

// Classes 0 and 1 are held to 4 waves per SIMD (128 VGPRs).  Every class
// keeps its run partial in LDS (rows of at most 2048, 5120 and 12288
// elements) and stores it once per run.  The clip's second run partial is
// kept in LDS too in class 0, accumulated in the workspace in class 1 (in
// registers it would cost class 1 a wave per SIMD, measured slower) and kept
// in registers in class 2, whose LDS already limits it to 2 waves per SIMD.
template <int CLS, int EPS>
__global__ __launch_bounds__(KAON_WG, 4) void k_pf_stats(const KaonTensor* __restrict__ D,
                                                         const KaonItem* __restrict__ items, Ws ws, KaonHyper hp,
                                                         int mode) {
  __shared__ __attribute__((aligned(16))) float seg[2][4][512];
  __shared__ __attribute__((aligned(16))) float racc[CLS == 0 ? 4 * 512 : 10 * 512];
  __shared__ __attribute__((aligned(16))) float racc2[CLS == 0 ? 4 * 512 : 1];
  pf_stats_run<CLS, EPS, false>(D, items, ws, hp, mode, seg, racc, CLS == 0 ? racc2 : nullptr);
}
template <int EPS>
__global__ __launch_bounds__(KAON_WG) void k_pf_stats_wide(const KaonTensor* __restrict__ D,
                                                           const KaonItem* __restrict__ items, Ws ws, KaonHyper hp,
                                                           int mode) {
  __shared__ __attribute__((aligned(16))) float seg[4][4][512];  // two buffer sets of two segments
  __shared__ __attribute__((aligned(16))) float racc[24 * 512];
  pf_stats_run<2, EPS, true>(D, items, ws, hp, mode, seg, racc, nullptr);
}

#undef KAON_PF_SWITCH
#undef KAON_COMMA

// =============================================================== phases 5/6
// Momentum chunk load (raw codes / bits) and store.
template <int CODEC>
__device__ __forceinline__ void ld_mom_at(const void* mbuf, int64_t e0, int cnt, bool vec, uint32_t q[8]) {
  if (CODEC == KAON_MOM_INT8) {
    const int8_t* m = (const int8_t*)mbuf + e0;
    if (vec) {
      const ku2 v = *(const KAON_G ku2*)G(m);
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
    // nibble of element e = byte e/2, low nibble for even e (any alignment)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i < cnt) {
        const int64_t e = e0 + i;
        q[i] = ((uint32_t)((const uint8_t*)mbuf)[e >> 1] >> (4 * (e & 1))) & 0xFu;
      } else {
        q[i] = 8u;
      }
    }
    (void)vec;
  } else if (CODEC == KAON_MOM_BF16) {
    ld8_bits(mbuf, e0, cnt, vec, q);
  } else if (CODEC == KAON_MOM_F32) {
    float f[8];
    ld8<KAON_F32>(mbuf, e0, cnt, vec, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = __float_as_uint(f[i]);
  }
}

template <int CODEC>
__device__ __forceinline__ void ld_mom_raw(const KaonTensor& T, int64_t e0, int cnt, bool vec, uint32_t q[8]) {
  ld_mom_at<CODEC>(T.m, e0, cnt, vec, q);
}

// n = the tensor's element count (the last byte of an odd-length 4-bit buffer)
template <int CODEC>
__device__ __forceinline__ void st_mom_at(void* mbuf, int64_t n, int64_t e0, int cnt, bool vec, const uint32_t q[8]) {
  if (CODEC == KAON_MOM_INT8) {
    int8_t* m = (int8_t*)mbuf + e0;
    if (vec) {
      ku2 v;
      v.x = (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | ((q[3] & 0xFF) << 24);
      v.y = (q[4] & 0xFF) | ((q[5] & 0xFF) << 8) | ((q[6] & 0xFF) << 16) | ((q[7] & 0xFF) << 24);
      *(KAON_G ku2*)G(m) = v;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < cnt) m[i] = (int8_t)q[i];
    }
  } else if (CODEC == KAON_MOM_4BIT) {
    uint8_t* m = (uint8_t*)mbuf;
    if (vec && (e0 & 7) == 0) {
      uint32_t v = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) v |= (q[i] & 0xFu) << (4 * i);
      *(uint32_t*)(m + (e0 >> 1)) = v;
    } else {
      // bytes shared with a neighbouring chunk (odd starts) are merged with an
      // atomic; the byte of an odd-length tensor's last element keeps 0 in its
      // high nibble (_pack_nibbles pads with 0)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i >= cnt) break;
        const int64_t e = e0 + i;
        const int sh = 4 * (int)(e & 1);
        uint32_t* word = (uint32_t*)(m + ((e >> 1) & ~(int64_t)3));
        const int bsh = 8 * (int)((e >> 1) & 3) + sh;
        // the last element of an odd-length tensor owns its whole byte
        const uint32_t clear = (e + 1 == n && (e & 1) == 0) ? 0xFFu : 0xFu;
        atomicAnd(word, ~(clear << bsh));
        atomicOr(word, (q[i] & 0xFu) << bsh);
      }
    }
  } else if (CODEC == KAON_MOM_BF16) {
    st8_bits(mbuf, e0, cnt, vec, q);
  } else if (CODEC == KAON_MOM_F32) {
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(q[i]);
    st8_f32(mbuf, e0, cnt, vec, f);
  }
}

template <int CODEC>
__device__ __forceinline__ void st_mom_raw(const KaonTensor& T, int64_t e0, int cnt, bool vec, const uint32_t q[8]) {
  st_mom_at<CODEC>(T.m, T.n, e0, cnt, vec, q);
}

// int8 dequant q*sc with q the stored byte: (ub - 128)*sc = fma(ub, sc, -128 sc)
// with ub = byte ^ 0x80, exact because 128*sc is exact (no overflow below 2^120).
__device__ __forceinline__ float dq_int8(uint32_t byte, float sc, float m128sc, bool fast) {
  if (fast) return __fmaf_rn((float)((byte ^ 0x80u) & 0xFFu), sc, m128sc);
  return (float)(int8_t)(uint8_t)byte * sc;
}

// The |m| maxima of 4-bit blocks that cross chunks or rows: the elements a
// thread visits in one block are reduced in registers and stored with one
// atomic per run (NaN never enters: fmaxf keeps its other operand, as the
// per-element form skipped NaN).
struct BlkMax {
  uint32_t blk = 0xFFFFFFFFu;
  float mx = 0.0f;
  __device__ __forceinline__ void flush(KAON_G uint32_t* bamax) {
    if (blk != 0xFFFFFFFFu && mx > 0.0f) atomicMax((uint32_t*)&bamax[blk], __float_as_uint(mx));
  }
  __device__ __forceinline__ void add(KAON_G uint32_t* bamax, uint32_t b, float ax) {
    if (b != blk) {
      flush(bamax);
      blk = b;
      mx = 0.0f;
    }
    mx = fmaxf(mx, ax);
  }
};

// =============================================================== AdaMuon momentum
// The first moment of the raw gradient (adamuon.py:570-573 via the codecs'
// ema_one, _momentum_codec.py:266-269, 303-308, 363-371): M = lerp(m, g, 1 -
// beta1) (g centralized first when GC is on), written as bf16 into the
// Newton-Schulz block.  Float codecs store m here; int8 / 4-bit record the
// row / block absmax and the old scales, and phase 6 requantizes M with them.
// Also: the GC means (phases 5 and 6 use them), and each row's sum of M^2 for
// the Frobenius norm of the Newton-Schulz input.

// 4-bit block absmax is accumulated with atomics: clear it (one tensor per
// workgroup) before the momentum pass.
__global__ __launch_bounds__(KAON_WG) void k_muon_zero(const KaonTensor* __restrict__ D, int32_t n_tensors, Ws ws) {
  const KaonTensor& T = D[blockIdx.x];
  const int64_t nb = nblocks4(T);
  for (int64_t b = threadIdx.x; b < nb; b += KAON_WG) ws.bamax(T)[b] = 0u;
}

template <int GT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_muon_mom(const KaonTensor* __restrict__ D,
                                                      const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C;
  const int64_t nch = (C + 7) >> 3;
  const int cpl = (int)((nch + 63) >> 6);
  const bool vec = T.vec_rows != 0;
  const bool gc = (hp.flags & KAON_F_GC) != 0;
  const bool mom = (hp.flags & KAON_F_MOMENTUM) != 0 && CODEC != KAON_MOM_NONE;
  const int64_t B = CODEC == KAON_MOM_4BIT ? (int64_t)T.block4 : 1;
  const int64_t nb = CODEC == KAON_MOM_4BIT ? nblocks4(T) : 0;
  KAON_G uint16_t* mo = G(ws.mo(T));
  const int nsl = run_slices(it);
#pragma clang loop unroll(disable)
  for (int sl = 0; sl < nsl; ++sl) {
  const WaveRows wr = wave_rows(slice_item(it, sl));
  for (int64_t r = wr.rb; r < wr.re; ++r) {
    float mu = 0.0f;
    if (gc) {
      float a = 0.0f;
      for (int k = 0; k < cpl; ++k) {
        const int64_t c = wr.lane + 64 * k;
        const int cnt = chunk_cnt(c, C);
        if (cnt <= 0) continue;
        float x[8];
        ld8<GT>(T.g, r * C + c * 8, cnt, vec && cnt == 8, x);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i < cnt) a = a + x[i];
      }
      mu = round_to<GT>(wave_csum(a) / (float)C);
      if (wr.lane == 0) ws.mu(T)[r] = mu;
    }
    const float oldsc = CODEC == KAON_MOM_INT8 && mom ? uniform_f(G(T.m_scale)[r]) : 1.0f;
    float amax = 0.0f, sq = 0.0f;
    BlkMax bm4;
    for (int k = 0; k < cpl; ++k) {
      const int64_t c = wr.lane + 64 * k;
      const int cnt = chunk_cnt(c, C);
      if (cnt <= 0) continue;
      const int64_t e0 = r * C + c * 8;
      const bool vv = vec && cnt == 8;
      float g[8];
      ld8<GT>(T.g, e0, cnt, vv, g);
      if (gc) {
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = round_to<GT>(g[i] - mu);
      }
      uint32_t mq[8];
      if (mom) ld_mom_raw<CODEC>(T, e0, cnt, vv, mq);
      uint32_t qout[8], mob[8];
      float Mv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qout[i] = 0u;
        mob[i] = 0u;
        Mv[i] = 0.0f;
        if (i >= cnt) continue;
        if (!mom) {
          Mv[i] = g[i];
        } else if (CODEC == KAON_MOM_BF16) {
          const uint32_t mb = f2bf(klerp(bf2f(mq[i]), rbf(g[i]), hp.w1));
          qout[i] = mb;
          Mv[i] = bf2f(mb);
        } else if (CODEC == KAON_MOM_F32) {
          Mv[i] = klerp(__uint_as_float(mq[i]), g[i], hp.w1);
          qout[i] = __float_as_uint(Mv[i]);
        } else if (CODEC == KAON_MOM_INT8) {
          Mv[i] = klerp(dq_int8(mq[i], oldsc, -128.0f * oldsc, fabsf(oldsc) < 0x1p120f), g[i], hp.w1);
          amax = fmaxf(amax, fabsf(Mv[i]));
        } else {  // 4-bit: flat blocks, possibly across rows (32-bit: n < 2^31)
          const uint32_t e = (uint32_t)e0 + (uint32_t)i, blk = e / (uint32_t)B;
          const float sc = G(T.m_scale)[blk];
          Mv[i] = klerp(((float)mq[i] - 8.0f) * sc, g[i], hp.w1);
          bm4.add(ws.bamax(T), blk, fabsf(Mv[i]));
          if (e == blk * (uint32_t)B) ws.boldsc(T, nb)[blk] = sc;
        }
        const uint32_t xb = f2bf(Mv[i]);
        const float xf = bf2f(xb);
        sq = sq + xf * xf;
        mob[i] = xb;
      }
      if (vv) {
        *(KAON_G ku4*)(mo + e0) = ku4{mob[0] | (mob[1] << 16), mob[2] | (mob[3] << 16), mob[4] | (mob[5] << 16),
                                      mob[6] | (mob[7] << 16)};
      } else {
        for (int i = 0; i < cnt; ++i) mo[e0 + i] = (uint16_t)mob[i];
      }
      if (mom && (CODEC == KAON_MOM_BF16 || CODEC == KAON_MOM_F32)) st_mom_raw<CODEC>(T, e0, cnt, vv, qout);
    }
    if (CODEC == KAON_MOM_4BIT) bm4.flush(ws.bamax(T));
    if (CODEC == KAON_MOM_INT8 && mom) {
      const float am = wave_max(amax);
      if (wr.lane == 0) {
        ws.ramax(T)[r] = __float_as_uint(am);
        ws.roldsc(T)[r] = oldsc;
      }
    }
    const float s2 = wave_csum(sq);
    if (wr.lane == 0) ws.rs(T)[r] = s2;
  }
  }
}

// den = bf16(bf16(||M||) + 1e-7) per tensor (x.norm() + 1e-7 on bf16 tensors,
// adamuon.py:109), one wave per tensor, stored in the tensor's spare scalar.
__global__ __launch_bounds__(KAON_WG) void k_muon_norm(const KaonTensor* __restrict__ D, int32_t n_tensors, Ws ws) {
  const int t = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (t >= n_tensors) return;
  const KaonTensor& T = D[t];
  const int lane = threadIdx.x & 63;
  const KAON_G float* rs = ws.rs(T);
  float a = 0.0f;
  for (int64_t r = lane; r < T.R; r += 64) a = a + rs[r];
  const float ss = wave_csum(a);
  if (lane == 0) ws.scal(T)[2] = rbf(rbf(sqrtf(ss)) + 1e-7f);
}

// Per-chunk body of phases 5 and 6.  Row context (mu, rf, scales) is uniform
// over the chunk when `one_row`; otherwise it is looked up per element.
struct RowCtx {
  float mu, rf, oldsc, newsc, m128, m128n;
  double rnew;
  bool fast;
};

// A row value read once per row: wave-uniform (a scalar) when the wave works
// on one row at a time, per lane when it packs several rows.
template <bool PK>
__device__ __forceinline__ float row_val(float x) {
  return PK ? x : uniform_f(x);
}

// The rows of a wave's share of a slice, phases 5 and 6, in one of three
// layouts.  LAY 0: one row at a time, lane l taking chunks l, l+64, ....
// LAY 1 (rows of at most 32 chunks): L = 2^ceil(log2(chunks)) lanes per row,
// 64 / L rows side by side, lane cl of a row's lane group taking chunk cl.
// LAY 2 (an item of one row, e.g. a 1-D tensor): the four waves share the row,
// wave w taking the chunk rounds w, w+4, ... of LAY 0.  Every element's
// arithmetic is the same in all three; the only reductions across lanes are
// the keep count (an integer sum), the int8 row absmax and the 4-bit block
// absmax (maxima; blocks that cross chunks go through atomicMax), none of
// which depends on the order.  Returns the lane's keep count.
template <int OPT, int PHASE, int PT, int GT, int CODEC, int LAY>
__device__ __forceinline__ uint32_t elem_rows(const KaonTensor& T, const KaonItem& it, const Ws& ws,
                                              const KaonHyper& hp) {
  const int64_t C = T.C, n = T.n;
  const int64_t nch = (C + 7) >> 3;
  const int cpl = (int)((nch + 63) >> 6);
  const bool vec_t = T.vec_rows != 0;
  const bool factored = T.factored != 0;
  const bool gc = (hp.flags & KAON_F_GC) && factored;
  const bool cautious = (hp.flags & KAON_F_CAUTIOUS) != 0;
  const bool wd = (hp.flags & KAON_F_WD) != 0;
  constexpr bool MUON = OPT == KAON_OPT_ADAMUON;
  constexpr bool QUANT_C = CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT;
  // AdaMuon's momentum is the raw grad's: float codecs were stored by the
  // momentum pass; int8 / 4-bit codes are requantized here in phase 6
  const bool mom = (hp.flags & KAON_F_MOMENTUM) != 0 && CODEC != KAON_MOM_NONE && (!MUON || (PHASE == 6 && QUANT_C));
  const bool nk_remove = OPT == KAON_OPT_ADAKAON && mom && (hp.flags & KAON_F_NK_REMOVE);
  const bool nk_climb = OPT == KAON_OPT_ADAKAON && mom && (hp.flags & KAON_F_NK_CLIMB);
  const float nf_old = msam_nanfill(hp.nk_bound_old), nf_new = msam_nanfill(hp.nk_bound_new);
  constexpr bool QUANT = CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT;
  const bool quant = mom && QUANT;
  const bool lowp = PT == KAON_BF16;
  const int64_t B = CODEC == KAON_MOM_4BIT ? (int64_t)T.block4 : 1;
  const int64_t nb = CODEC == KAON_MOM_4BIT ? nblocks4(T) : 0;
  const WaveRows wr = wave_rows(it);

  // clip divisor of the tensor (phase 4)
  const float fac = OPT != KAON_OPT_LION ? ws.scal(T)[0] : 1.0f;
  const double rfac = rcp64(fac);
  double rden = 1.0;
  if (PHASE == 6 && cautious) {
    const uint32_t cnt = ((const KAON_G uint32_t*)ws.scal(T))[1];
    rden = rcp64(fmaxf((float)cnt / (float)n, 1e-8f));
  }
  // 4-bit fast path: blocks inside rows, a block = G consecutive chunks = G lanes
  const int64_t GL = CODEC == KAON_MOM_4BIT && B >= 8 ? B / 8 : 1;
  const bool blk_fast = CODEC == KAON_MOM_4BIT && B % 8 == 0 && C % B == 0 && GL <= 64 && (64 % GL) == 0 && vec_t;
  uint32_t keep = 0;
  BlkMax bm4;  // 4-bit blocks across chunks or rows (phase 5)
  // the scales of the last 4-bit block visited (blocks across chunks or rows):
  // read once per run of a block's elements
  uint32_t c_blk = 0xFFFFFFFFu;
  float c_old = 1.0f, c_new = 1.0f;
  double c_r = 1.0;
  // lanes per row (2^lsh) and rows side by side (P); the lane's row in a pass
  // and its chunk
  constexpr bool PK = LAY == 1;
  const int lsh = PK ? (nch <= 1 ? 0 : 32 - __builtin_clz((uint32_t)(nch - 1))) : 6;
  const int P = 64 >> lsh;
  const int grp = wr.lane >> lsh;
  const int cl = wr.lane & ((1 << lsh) - 1);
  // the lane that stores the row's values (LAY 2: of wave 0)
  const bool lead = cl == 0 && (LAY != 2 || wr.w == 0);
  // the rows and the chunk rounds of this wave
  const int64_t rbeg = LAY == 2 ? (int64_t)it.row0 : wr.rb;
  const int64_t rend = LAY == 2 ? (int64_t)it.row0 + 1 : wr.re;
  const int k0 = LAY == 2 ? wr.w : 0;
  constexpr int kstep = LAY == 2 ? 4 : 1;

  for (int64_t r0 = rbeg; r0 < rend; r0 += P) {
    // the lane's row; lanes past the wave's rows read the first row's context
    // and take no chunk
    const bool rvalid = r0 + grp < rend;
    const int64_t r = rvalid ? r0 + grp : rbeg;
    // ---- per-row context (wave-uniform unless PK)
    RowCtx rc;
    rc.mu = gc ? row_val<PK>(ws.mu(T)[r]) : 0.0f;
    rc.rf = (OPT != KAON_OPT_LION && factored) ? row_val<PK>(ws.rf(T)[r]) : 0.0f;
    rc.oldsc = 1.0f;
    rc.newsc = 1.0f;
    rc.rnew = 1.0;
    if (CODEC == KAON_MOM_INT8 && mom) {
      rc.oldsc = row_val<PK>(PHASE == 5 ? T.m_scale[r] : ws.roldsc(T)[r]);
      if (PHASE == 6) {
        rc.newsc = row_val<PK>(fmaxf(__uint_as_float(ws.ramax(T)[r]), 1e-12f) / 127.0f);
        rc.rnew = rcp64(rc.newsc);
      }
    }
    rc.fast = fabsf(rc.oldsc) < 0x1p120f && fabsf(rc.newsc) < 0x1p120f;
    rc.m128 = -128.0f * rc.oldsc;
    float row_amax = 0.0f;

    for (int k = k0; k < cpl; k += kstep) {
      const int64_t c = cl + 64 * k;
      const int cnt = rvalid ? chunk_cnt(c, C) : 0;
      const int64_t j0 = c * 8;
      const int64_t e0 = r * C + j0;
      const bool vec = vec_t && cnt == 8;
      // ---- loads
      float g[8], p[8], f[8];
      uint32_t mq[8], pb[8];
      if (cnt > 0) {
        ld8<GT>(T.g, e0, cnt, vec, g);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = 0.0f;
      }
      const bool need_p = PHASE == 6 || wd;
      if (need_p && cnt > 0) {
        if (PT != KAON_F32) {
          ld8_bits(T.p, e0, cnt, vec, pb);
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = lp2f<PT>(pb[i]);
        } else {
          ld8<KAON_F32>(T.p, e0, cnt, vec, p);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = 0.0f;
      }
      if (mom && cnt > 0) ld_mom_raw<CODEC>(T, e0, cnt, vec, mq);
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) mq[i] = CODEC == KAON_MOM_4BIT ? 8u : 0u;
      float ov[8];
      if (MUON && cnt > 0) ld8<KAON_BF16>(ws.mo(T), e0, cnt, vec, ov);
      if (OPT != KAON_OPT_LION && cnt > 0) {
        if (factored) ld8<KAON_F32>((const float*)ws.cf(T), j0, cnt, vec, f);
        else ld8<KAON_F32>(T.v, j0, cnt, vec, f);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = 1.0f;
      }
      // 4-bit block scales: one block per chunk on the fast path
      float b_old = 1.0f, b_new = 1.0f;
      double b_rnew = 1.0;
      int64_t blk = 0;
      if (CODEC == KAON_MOM_4BIT && mom && blk_fast) {
        blk = e0 / B;
        if (cnt > 0) {
          b_old = PHASE == 5 ? T.m_scale[blk] : ws.boldsc(T, nb)[blk];
          if (PHASE == 6) {
            b_new = fmaxf(__uint_as_float(ws.bamax(T)[blk]), 1e-12f) / 7.0f;
            b_rnew = rcp64(b_new);
          }
        }
      }
      // ---- noise (phase 6, bf16 weights)
      uint32_t nz0[8], nz1[8], nz2[8];
      if (lowp && cnt > 0) {
        const bool aligned = (e0 & 7) == 0;
        if (nk_remove && need_p) {
          if (aligned) noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 0u, e0, T.noise[0], cnt, nz0);
          else
#pragma unroll
            for (int i = 0; i < 8; ++i) nz0[i] = i < cnt ? noise1(hp.seed, hp.step, T.tensor_id, 0u, e0 + i, T.noise[0]) : 0u;
        }
        if (PHASE == 6 && hp.bf16_method == KAON_SR) {
          if (aligned) noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 1u, e0, T.noise[1], cnt, nz1);
          else
#pragma unroll
            for (int i = 0; i < 8; ++i) nz1[i] = i < cnt ? noise1(hp.seed, hp.step, T.tensor_id, 1u, e0 + i, T.noise[1]) : 0u;
        }
        if (PHASE == 6 && nk_climb) {
          if (aligned) noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 2u, e0, T.noise[2], cnt, nz2);
          else
#pragma unroll
            for (int i = 0; i < 8; ++i) nz2[i] = i < cnt ? noise1(hp.seed, hp.step, T.tensor_id, 2u, e0 + i, T.noise[2]) : 0u;
        }
      }
      // ---- gradient as the step sees it (GC in the grad dtype)
      if (gc) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          float a0 = g[i] - rc.mu, a1 = g[i + 1] - rc.mu;
          round_pair<GT>(a0, a1);
          g[i] = a0;
          g[i + 1] = a1;
        }
      }
      // ---- per element
      uint32_t qout[8];
      float dout[8], mnew[8];
      float chunk_amax = 0.0f;
      // 4-bit blocks that cross chunks or rows: the chunk's first block and offset
      // (one 32-bit division, n < 2^32), then walked element by element
      uint32_t wblk = 0u, woff = 0u;
      if (CODEC == KAON_MOM_4BIT && mom && !blk_fast) {
        wblk = (uint32_t)e0 / (uint32_t)B;
        woff = (uint32_t)e0 - wblk * (uint32_t)B;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qout[i] = mq[i];
        dout[i] = 0.0f;
        mnew[i] = 0.0f;
        if (i >= cnt) continue;
        float sc4_old = b_old, sc4_new = b_new;
        double r4 = b_rnew;
        int64_t blk_e = blk;
        bool blk_first = false;  // the element opens its block
        if (CODEC == KAON_MOM_4BIT && mom && !blk_fast) {
          blk_e = wblk;
          blk_first = woff == 0u;
          if (++woff == (uint32_t)B) {
            woff = 0u;
            ++wblk;
          }
          if ((uint32_t)blk_e != c_blk) {
            c_blk = (uint32_t)blk_e;
            c_old = PHASE == 5 ? T.m_scale[blk_e] : ws.boldsc(T, nb)[blk_e];
            if (PHASE == 6) {
              c_new = fmaxf(__uint_as_float(ws.bamax(T)[blk_e]), 1e-12f) / 7.0f;
              c_r = rcp64(c_new);
            }
          }
          sc4_old = c_old;
          sc4_new = c_new;
          r4 = c_r;
        }
        float mold = 0.0f;
        if (mom) {
          if (CODEC == KAON_MOM_INT8) mold = dq_int8(mq[i], rc.oldsc, rc.m128, rc.fast);
          else if (CODEC == KAON_MOM_4BIT) mold = ((float)mq[i] - 8.0f) * sc4_old;
          else if (CODEC == KAON_MOM_BF16) mold = bf2f(mq[i]);
          else if (CODEC == KAON_MOM_F32) mold = __uint_as_float(mq[i]);
        }
        float pw = p[i];  // weight the inner step sees (after the Nekaon removal)
        if (nk_remove && need_p) {
          const float ev = msam_e(mold * hp.nk_k, hp.nk_bound_old, nf_old);
          pw = lowp ? bf2f(sr_bf16(p[i] + ev, nz0[i])) : p[i] + ev;
        }
        float d, mfv = 0.0f;
        const float gv = g[i];
        if (OPT == KAON_OPT_ADAKAON) {
          const float u = factored ? (gv * rc.rf) * f[i] : gv * (1.0f / sqrtf(f[i]));
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
        } else if (MUON) {
          // U = O * r * c, clipped, times 0.2*lr (hp.lr); the momentum update
          // is of the grad (requantized below)
          const float u = (ov[i] * rc.rf) * f[i];
          d = (fac == 1.0f ? u : div_r64(u, rfac)) * hp.lr;
          if (mom) mfv = klerp(mold, gv, hp.w1);
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
            const float ax = fabsf(mfv);
            if (CODEC == KAON_MOM_4BIT && !blk_fast) {
              bm4.add(ws.bamax(T), (uint32_t)blk_e, ax);
              if (blk_first) ws.boldsc(T, nb)[blk_e] = sc4_old;
            } else {
              chunk_amax = fmaxf(chunk_amax, ax);
            }
          }
        } else {
          float mdeq = 0.0f;
          if (quant) {
            if (CODEC == KAON_MOM_INT8) {
              float x = rintf(div_r64(mfv, rc.rnew));
              x = fminf(fmaxf(x, -127.0f), 127.0f);
              qout[i] = (uint32_t)(uint8_t)(int8_t)x;
              mdeq = x * rc.newsc;
            } else {
              float x = rintf(div_r64(mfv, r4));
              x = fminf(fmaxf(x, -7.0f), 7.0f);
              qout[i] = (uint32_t)((int)x + 8);
              mdeq = x * sc4_new;
              if (!blk_fast && blk_first) T.m_scale[blk_e] = sc4_new;
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
      }

      if (PHASE == 5) {
        if (quant && !(CODEC == KAON_MOM_4BIT && !blk_fast)) {
          if (CODEC == KAON_MOM_INT8) {
            row_amax = fmaxf(row_amax, chunk_amax);
          } else {
            // blocks of G lanes: reduce within the lane group, its first lane stores
            float a = chunk_amax;
            for (int o = (int)GL / 2; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
            if (cnt > 0 && (wr.lane % GL) == 0) {
              ws.bamax(T)[blk] = __float_as_uint(a);
              ws.boldsc(T, nb)[blk] = b_old;
            }
          }
        }
        continue;
      }
      if (cnt <= 0) continue;
      // ---------------- phase 6 writes
      if (gc && (hp.flags & KAON_F_GC_WRITE) && T.gc_write && (OPT == KAON_OPT_ADAKAON || OPT == KAON_OPT_LION)) {
        // the centralized gradient over p.grad (already rounded to the grad dtype)
        if (GT == KAON_F32) {
          st8_f32(const_cast<void*>(T.g), e0, cnt, vec, g);
        } else {
          uint32_t gb[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) gb[i] = f2lp<GT>(g[i]);
          st8_bits(const_cast<void*>(T.g), e0, cnt, vec, gb);
        }
      }
      if (CODEC == KAON_MOM_4BIT && mom && blk_fast && (wr.lane % GL) == 0) G(T.m_scale)[blk] = b_new;
      if (mom) st_mom_raw<CODEC>(T, e0, cnt, vec, qout);
      if (PT == KAON_F32) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float x = p[i] - dout[i];
          if (nk_climb) x = x + msam_e(mnew[i] * (-hp.nk_k), hp.nk_bound_new, nf_new);
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
            // shift -= lp(delta); p0 = p; p += shift; shift += p0 - p, in the
            // param dtype (_backend.py:90-94)
            const float s = round_to<PT>(lp2f<PT>(sh[i]) - round_to<PT>(dout[i]));
            const float p0 = p[i];
            const float p1 = round_to<PT>(p0 + s);
            o[i] = f2lp<PT>(p1);
            sh[i] = f2lp<PT>(s + round_to<PT>(p0 - p1));
          }
          st8_bits(T.shift, e0, cnt, vec, sh);
        } else if (hp.bf16_method == KAON_RN || PT == KAON_F16) {
          // fp16 params are written by RN under "stochastic_rounding" too: the
          // reference's SR write is bf16-only (_backend.py:95-98)
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = f2lp<PT>(p[i] - round_to<PT>(dout[i]));
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = sr_bf16(p[i] - dout[i], nz1[i]);
        }
        if (nk_climb) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            o[i] = sr_bf16(bf2f(o[i]) + msam_e(mnew[i] * (-hp.nk_k), hp.nk_bound_new, nf_new), nz2[i]);
        }
        st8_bits(T.p, e0, cnt, vec, o);
      }
    }
    // ---- end of row
    if (CODEC == KAON_MOM_INT8 && quant) {
      if (PHASE == 5) {
        float am;
        if (PK) {
          // the maximum over the row's lane group (the other lanes of a
          // 64-lane row hold 0, which a maximum of |m| ignores)
          am = row_amax;
          for (int o = (1 << lsh) >> 1; o >= 1; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
        } else {
          am = wave_max(row_amax);
          if (LAY == 2) {
            // the four waves' maxima (every wave is here: the row is the item's)
            __shared__ float wmax[4];
            if (wr.lane == 0) wmax[wr.w] = am;
            __syncthreads();
            am = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
          }
        }
        if (rvalid && lead) {
          ws.ramax(T)[r] = __float_as_uint(am);
          ws.roldsc(T)[r] = rc.oldsc;
        }
      } else if (rvalid && lead) {
        T.m_scale[r] = rc.newsc;
      }
    }
  }

  if (PHASE == 5 && CODEC == KAON_MOM_4BIT) bm4.flush(ws.bamax(T));
  return keep;
}

template <int OPT, int PHASE, int PT, int GT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_elem(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ uint32_t keep_s[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const bool cautious = (hp.flags & KAON_F_CAUTIOUS) != 0;
  uint32_t keep;
  // rows of at most 32 chunks side by side (4-bit blocks are walked row by
  // row); an item of one row over the four waves; otherwise a row per wave
  bool done = false;
  if constexpr (CODEC != KAON_MOM_4BIT) {
    if (((T.C + 7) >> 3) <= 32) {
      keep = elem_rows<OPT, PHASE, PT, GT, CODEC, 1>(T, it, ws, hp);
      done = true;
    }
  }
  if (!done) {
    if (it.nrows == 1) keep = elem_rows<OPT, PHASE, PT, GT, CODEC, 2>(T, it, ws, hp);
    else keep = elem_rows<OPT, PHASE, PT, GT, CODEC, 0>(T, it, ws, hp);
  }
  if (PHASE == 5 && cautious) {
    const uint32_t wsum = wave_sum_u32(keep);
    const WaveRows wr = wave_rows(it);
    if (wr.lane == 0) keep_s[wr.w] = wsum;
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t tot = keep_s[0] + keep_s[1] + keep_s[2] + keep_s[3];
      if (tot) atomicAdd(ws.keep_ctr(T), tot);
    }
  }
}

// =============================================================== AdaPNM
// Phases 3, 5 and 6 of AdaPNM (_step_one_param, adapnm.py:1209-1275), per
// element with g the (centralized) gradient:
//   m_pos' = fma(1 - b1^2, g, m_pos * b1^2)       this step's positive buffer
//   pn     = fma(-b0, m_neg, m_pos' * (1 + b0)) * (1 / noise_norm)
//   u      = pn * ((r * c) * bc2)                   factored
//          = pn / ((sqrt(v + 1e-15) + eps) / bc2)   1-D (max_v under ams_bound)
//   d      = (u / fac) * lr / (1 - b1^t)
// Phase 3 (slices of row runs): the row sums of u^2 for the clip, and the
// absmax of m_pos' per int8 row / 4-bit block with the old scales.  Phase 5:
// the cautious keep count of d * g > 0.  Phase 6: requantize or store m_pos',
// write p after the decoupled decay p * (1 - lr*wd).  The negative buffer is
// only read.  Odd steps take m as the positive buffer, even steps m2.
template <int PHASE, int PT, int GT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_pnm(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ uint32_t keep_s[4];
  KaonItem it;
  if (PHASE == 3) {
    const KaonItem run = items[blockIdx.x / KAON_RUN];
    const int sl = (int)(blockIdx.x % KAON_RUN);
    if (sl >= run_slices(run)) return;
    it = slice_item(run, sl);
  } else {
    it = items[blockIdx.x];
  }
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C, n = T.n;
  const int64_t nch = (C + 7) >> 3;
  const int cpl = (int)((nch + 63) >> 6);
  const bool vec_t = T.vec_rows != 0;
  const bool factored = T.factored != 0;
  const bool gc = (hp.flags & KAON_F_GC) && factored;
  const bool cautious = (hp.flags & KAON_F_CAUTIOUS) != 0;
  const bool wd = (hp.flags & KAON_F_WD) != 0;
  const bool ams = (hp.flags & KAON_F_AMS) && !factored && T.max_v;
  const bool lowp = PT == KAON_BF16;
  constexpr bool QUANT = CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT;
  const bool swap = (hp.step & 1u) == 0u;
  void* mpos = swap ? T.m2 : T.m;
  const void* mneg = swap ? T.m : T.m2;
  float* spos = swap ? T.m2_scale : T.m_scale;
  const float* sneg = swap ? T.m_scale : T.m2_scale;
  const int64_t B = CODEC == KAON_MOM_4BIT ? (int64_t)T.block4 : 1;
  const int64_t nb = CODEC == KAON_MOM_4BIT ? nblocks4(T) : 0;
  const WaveRows wr = wave_rows(it);
  const float fac = PHASE == 3 ? 1.0f : ws.scal(T)[0];
  const double rfac = rcp64(fac);
  double rden = 1.0;
  if (PHASE == 6 && cautious) {
    const uint32_t cnt = ((const KAON_G uint32_t*)ws.scal(T))[1];
    rden = rcp64(fmaxf((float)cnt / (float)n, 1e-8f));
  }
  const float* fsrc = factored ? (const float*)ws.cf(T) : (ams ? T.max_v : T.v);
  uint32_t keep = 0;
  BlkMax bm4;  // 4-bit blocks across chunks or rows (phase 3)
  // the scales of the last 4-bit block visited: read once per run of its elements
  uint32_t c_blk = 0xFFFFFFFFu;
  float c_o = 1.0f, c_g = 1.0f, c_n = 1.0f;
  double c_r = 1.0;

  for (int64_t r = wr.rb; r < wr.re; ++r) {
    const float mu = gc ? uniform_f(ws.mu(T)[r]) : 0.0f;
    const float rf = factored ? uniform_f(ws.rf(T)[r]) : 0.0f;
    // int8 per-row scales (one for a 1-D tensor): the positive buffer's old one
    // (phase 6: as phase 3 recorded it), its new one (phase 6), the negative one
    const int64_t sr = factored ? r : 0;
    float oldsc = 1.0f, newsc = 1.0f, negsc = 1.0f;
    double rnew = 1.0;
    if (CODEC == KAON_MOM_INT8) {
      oldsc = uniform_f(PHASE == 6 ? ws.roldsc(T)[r] : G(spos)[sr]);
      negsc = uniform_f(G(sneg)[sr]);
      if (PHASE == 6) {
        newsc = uniform_f(fmaxf(__uint_as_float(ws.ramax(T)[r]), 1e-12f) / 127.0f);
        rnew = rcp64(newsc);
      }
    }
    const bool dqf = fabsf(oldsc) < 0x1p120f && fabsf(negsc) < 0x1p120f;
    const float m128o = -128.0f * oldsc, m128n = -128.0f * negsc;
    float ss = 0.0f, row_amax = 0.0f;

    for (int k = 0; k < cpl; ++k) {
      const int64_t c = wr.lane + 64 * k;
      const int cnt = chunk_cnt(c, C);
      if (cnt <= 0) continue;
      const int64_t j0 = c * 8;
      const int64_t e0 = r * C + j0;
      const bool vec = vec_t && cnt == 8;
      float g[8], f[8], p[8];
      uint32_t mq[8], nq[8], pb[8];
      ld8<GT>(T.g, e0, cnt, vec, g);
      ld_mom_at<CODEC>(mpos, e0, cnt, vec, mq);
      ld_mom_at<CODEC>(mneg, e0, cnt, vec, nq);
      ld8<KAON_F32>(fsrc, j0, cnt, vec, f);
      if (PHASE == 6) {
        if (PT != KAON_F32) {
          ld8_bits(T.p, e0, cnt, vec, pb);
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = lp2f<PT>(pb[i]);
        } else {
          ld8<KAON_F32>(T.p, e0, cnt, vec, p);
        }
      }
      uint32_t nz[8];
      if (PHASE == 6 && lowp && hp.bf16_method == KAON_SR) {
        if ((e0 & 7) == 0) noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 1u, e0, T.noise[1], cnt, nz);
        else
#pragma unroll
          for (int i = 0; i < 8; ++i) nz[i] = i < cnt ? noise1(hp.seed, hp.step, T.tensor_id, 1u, e0 + i, T.noise[1]) : 0u;
      }
      if (gc) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          float a0 = g[i] - mu, a1 = g[i + 1] - mu;
          round_pair<GT>(a0, a1);
          g[i] = a0;
          g[i + 1] = a1;
        }
      }
      uint32_t qout[8];
      float dout[8];
      // 4-bit: the chunk's first block and offset (one 32-bit division, n < 2^31),
      // then walked element by element
      uint32_t wblk = 0u, woff = 0u;
      if (CODEC == KAON_MOM_4BIT) {
        wblk = (uint32_t)e0 / (uint32_t)B;
        woff = (uint32_t)e0 - wblk * (uint32_t)B;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qout[i] = mq[i];
        dout[i] = 0.0f;
        if (i >= cnt) continue;
        // 4-bit block scales of the element
        int64_t blk = 0;
        bool blk_first = false;  // the element opens its block
        float sc4o = 1.0f, sc4n = 1.0f, sc4g = 1.0f;
        double r4 = 1.0;
        if (CODEC == KAON_MOM_4BIT) {
          blk = wblk;
          blk_first = woff == 0u;
          if (++woff == (uint32_t)B) {
            woff = 0u;
            ++wblk;
          }
          if ((uint32_t)blk != c_blk) {
            c_blk = (uint32_t)blk;
            c_o = PHASE == 6 ? ws.boldsc(T, nb)[blk] : G(spos)[blk];
            c_g = G(sneg)[blk];
            if (PHASE == 6) {
              c_n = fmaxf(__uint_as_float(ws.bamax(T)[blk]), 1e-12f) / 7.0f;
              c_r = rcp64(c_n);
            }
          }
          sc4o = c_o;
          sc4g = c_g;
          sc4n = c_n;
          r4 = c_r;
        }
        float mold, mng;
        if (CODEC == KAON_MOM_INT8) {
          mold = dq_int8(mq[i], oldsc, m128o, dqf);
          mng = dq_int8(nq[i], negsc, m128n, dqf);
        } else if (CODEC == KAON_MOM_4BIT) {
          mold = ((float)mq[i] - 8.0f) * sc4o;
          mng = ((float)nq[i] - 8.0f) * sc4g;
        } else if (CODEC == KAON_MOM_BF16) {
          mold = bf2f(mq[i]);
          mng = bf2f(nq[i]);
        } else {
          mold = __uint_as_float(mq[i]);
          mng = __uint_as_float(nq[i]);
        }
        const float gv = g[i];
        const float mfv = __fmaf_rn(hp.a1, gv, mold * hp.b1);
        const float pn = __fmaf_rn(hp.pn_neg, mng, mfv * hp.pn_pos) * hp.pn_rnorm;
        const float u = factored ? pn * ((rf * f[i]) * hp.bc2) : pn / ((sqrtf(f[i] + 1e-15f) + hp.eps1) / hp.bc2);
        if (PHASE == 3) {
          ss = ss + u * u;
          if (QUANT) {
            const float ax = fabsf(mfv);
            if (CODEC == KAON_MOM_INT8) {
              row_amax = fmaxf(row_amax, ax);
            } else {
              bm4.add(ws.bamax(T), (uint32_t)blk, ax);
              if (blk_first) ws.boldsc(T, nb)[blk] = sc4o;
            }
          }
          continue;
        }
        const float d = (fac == 1.0f ? u : div_r64(u, rfac)) * hp.lr;
        const bool kp = d * gv > 0.0f;
        if (PHASE == 5) {
          keep += kp ? 1u : 0u;
          continue;
        }
        if (CODEC == KAON_MOM_INT8) {
          float x = rintf(div_r64(mfv, rnew));
          x = fminf(fmaxf(x, -127.0f), 127.0f);
          qout[i] = (uint32_t)(uint8_t)(int8_t)x;
        } else if (CODEC == KAON_MOM_4BIT) {
          float x = rintf(div_r64(mfv, r4));
          x = fminf(fmaxf(x, -7.0f), 7.0f);
          qout[i] = (uint32_t)((int)x + 8);
          if (blk_first) G(spos)[blk] = sc4n;
        } else if (CODEC == KAON_MOM_BF16) {
          qout[i] = f2bf(mfv);
        } else {
          qout[i] = __float_as_uint(mfv);
        }
        dout[i] = cautious ? div_r64(d * (kp ? 1.0f : 0.0f), rden) : d;
        // p.data.mul_(1 - lr*wd) in the param dtype (adapnm.py:1227-1228)
        if (wd) p[i] = round_to<PT>(p[i] * hp.wdl);
      }
      if (PHASE != 6) continue;
      // ---------------- phase 6 writes
      st_mom_at<CODEC>(mpos, n, e0, cnt, vec, qout);
      if (PT == KAON_F32) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = p[i] - dout[i];
        st8_f32(T.p, e0, cnt, vec, o);
      } else {
        uint32_t o[8];
        if (hp.bf16_method == KAON_KAHAN) {
          uint32_t sh[8];
          ld8_bits(T.shift, e0, cnt, vec, sh);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            // kahan in the param dtype (_backend.py:90-94)
            const float s = round_to<PT>(lp2f<PT>(sh[i]) - round_to<PT>(dout[i]));
            const float p0 = p[i];
            const float p1 = round_to<PT>(p0 + s);
            o[i] = f2lp<PT>(p1);
            sh[i] = f2lp<PT>(s + round_to<PT>(p0 - p1));
          }
          st8_bits(T.shift, e0, cnt, vec, sh);
        } else if (hp.bf16_method == KAON_RN || PT == KAON_F16) {
          // fp16 params take RN under "stochastic_rounding" too (_backend.py:95-98)
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = f2lp<PT>(p[i] - round_to<PT>(dout[i]));
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = sr_bf16(p[i] - dout[i], nz[i]);
        }
        st8_bits(T.p, e0, cnt, vec, o);
      }
    }
    // ---- end of row
    if (PHASE == 3) {
      const float s2 = wave_csum(ss);
      if (CODEC == KAON_MOM_INT8) {
        const float am = wave_max(row_amax);
        if (wr.lane == 0) {
          ws.ramax(T)[r] = __float_as_uint(am);
          ws.roldsc(T)[r] = oldsc;
        }
      }
      if (wr.lane == 0) ws.rs(T)[r] = s2;
    } else if (PHASE == 6 && CODEC == KAON_MOM_INT8 && wr.lane == 0) {
      G(spos)[sr] = newsc;
    }
  }

  if (PHASE == 3 && CODEC == KAON_MOM_4BIT) bm4.flush(ws.bamax(T));
  if (PHASE == 5 && cautious) {
    const uint32_t wsum = wave_sum_u32(keep);
    if (wr.lane == 0) keep_s[wr.w] = wsum;
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t tot = keep_s[0] + keep_s[1] + keep_s[2] + keep_s[3];
      if (tot) atomicAdd(ws.keep_ctr(T), tot);
    }
  }
}

// AdaPNM phase 3 on row class 0 (factored, bf16 g, 16-byte rows with
// C % 8 == 0, at most 4 chunks per lane) with int8 or bf16 momenta: the same
// arithmetic and 64-lane row order as k_pnm<3>, with all loads of a group of
// GR rows (g and both momenta, every chunk of the lane) issued before the
// group's arithmetic, and the per-row values read once per wave (one row per
// lane, then read across lanes).  Addresses are clamped to valid rows and
// chunks, so every load is unconditional.
template <int CPL, int GR, int CODEC>
__device__ __forceinline__ void pnm_ss_body(const KaonTensor& T, const KaonItem& it, const Ws& ws,
                                            const KaonHyper& hp) {
  constexpr bool I8 = CODEC == KAON_MOM_INT8;
  const uint32_t C = (uint32_t)T.C;
  const int nch = (int)(C >> 3);
  const WaveRows wr = wave_rows(it);
  const int nrows = (int)(wr.re - wr.rb);
  if (nrows <= 0) return;
  const bool gc = (hp.flags & KAON_F_GC) != 0;
  const bool swap = (hp.step & 1u) == 0u;
  const KAON_G uint8_t* mpos = (const KAON_G uint8_t*)G(swap ? T.m2 : T.m);
  const KAON_G uint8_t* mneg = (const KAON_G uint8_t*)G(swap ? T.m : T.m2);
  const KAON_G float* spos = G(swap ? T.m2_scale : T.m_scale);
  const KAON_G float* sneg = G(swap ? T.m_scale : T.m2_scale);
  const KAON_G uint8_t* gb = (const KAON_G uint8_t*)G(T.g);
  const KAON_G uint8_t* cfb = (const KAON_G uint8_t*)ws.cf(T);
  const int64_t rl = lane_row(wr.rb, nrows, wr.lane);
  const float mu_l = gc ? ws.mu(T)[rl] : 0.0f;
  const float rf_l = ws.rf(T)[rl];
  const float so_l = I8 ? spos[rl] : 1.0f;
  const float sn_l = I8 ? sneg[rl] : 1.0f;
  kf4 cfv[CPL][2];  // the column factors of the lane's chunks, held for the wave
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const uint32_t cb = 32u * (uint32_t)min(wr.lane + 64 * k, nch - 1);
    cfv[k][0] = *(const KAON_G kf4*)(cfb + cb);
    cfv[k][1] = *(const KAON_G kf4*)(cfb + cb + 16u);
  }
  for (int j0 = 0; j0 < nrows; j0 += GR) {
    ku4 graw[GR][CPL], m16[GR][CPL], n16[GR][CPL];
    ku2 m8[GR][CPL], n8[GR][CPL];
#pragma unroll
    for (int j = 0; j < GR; ++j) {
      const uint32_t rowe = (uint32_t)(wr.rb + min(j0 + j, nrows - 1)) * C;
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        const uint32_t e0 = rowe + 8u * (uint32_t)min(wr.lane + 64 * k, nch - 1);
        graw[j][k] = ld_stream<true>((const KAON_G ku4*)(gb + 2u * e0));
        if (I8) {
          m8[j][k] = ld_stream<true>((const KAON_G ku2*)(mpos + e0));
          n8[j][k] = ld_stream<true>((const KAON_G ku2*)(mneg + e0));
        } else {
          m16[j][k] = ld_stream<true>((const KAON_G ku4*)(mpos + 2u * e0));
          n16[j][k] = ld_stream<true>((const KAON_G ku4*)(mneg + 2u * e0));
        }
      }
    }
#pragma unroll
    for (int j = 0; j < GR; ++j) {
      const int jj = j0 + j;
      if (jj >= nrows) continue;
      const float mu = lane_val(mu_l, jj), rf = lane_val(rf_l, jj);
      const float oldsc = lane_val(so_l, jj), negsc = lane_val(sn_l, jj);
      const bool dqf = fabsf(oldsc) < 0x1p120f && fabsf(negsc) < 0x1p120f;
      const float m128o = -128.0f * oldsc, m128n = -128.0f * negsc;
      float ss = 0.0f, amax = 0.0f;
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        if (wr.lane + 64 * k >= nch) continue;
        float g[8], mo[8], mn[8];
        unpack8(graw[j][k], g);
        if (gc) {
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            float a0 = g[i] - mu, a1 = g[i + 1] - mu;
            rbf2(a0, a1);
            g[i] = a0;
            g[i + 1] = a1;
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (I8) {
            const uint32_t wm = i < 4 ? m8[j][k].x : m8[j][k].y, wn = i < 4 ? n8[j][k].x : n8[j][k].y;
            mo[i] = dq_int8((wm >> (8 * (i & 3))) & 0xFFu, oldsc, m128o, dqf);
            mn[i] = dq_int8((wn >> (8 * (i & 3))) & 0xFFu, negsc, m128n, dqf);
          } else {
            const uint32_t wm[4] = {m16[j][k].x, m16[j][k].y, m16[j][k].z, m16[j][k].w};
            const uint32_t wn[4] = {n16[j][k].x, n16[j][k].y, n16[j][k].z, n16[j][k].w};
            mo[i] = (i & 1) ? __uint_as_float(wm[i >> 1] & 0xFFFF0000u) : __uint_as_float(wm[i >> 1] << 16);
            mn[i] = (i & 1) ? __uint_as_float(wn[i >> 1] & 0xFFFF0000u) : __uint_as_float(wn[i >> 1] << 16);
          }
        }
        const kf4 c0 = cfv[k][0], c1 = cfv[k][1];
        const float f[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float mfv = __fmaf_rn(hp.a1, g[i], mo[i] * hp.b1);
          const float pn = __fmaf_rn(hp.pn_neg, mn[i], mfv * hp.pn_pos) * hp.pn_rnorm;
          const float u = pn * ((rf * f[i]) * hp.bc2);
          ss = ss + u * u;
          if (I8) amax = fmaxf(amax, fabsf(mfv));
        }
      }
      const float s2 = wave_csum(ss);
      const int64_t r = wr.rb + jj;
      if (I8) {
        const float am = wave_max(amax);
        if (wr.lane == 0) {
          ws.ramax(T)[r] = __float_as_uint(am);
          ws.roldsc(T)[r] = oldsc;
        }
      }
      if (wr.lane == 0) ws.rs(T)[r] = s2;
    }
  }
}

// One slice per workgroup: workgroup b takes slice b % KAON_RUN of run b / KAON_RUN.
template <int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_pnm_ss(const KaonTensor* __restrict__ D,
                                                    const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  const KaonItem run = items[blockIdx.x / KAON_RUN];
  const int sl = (int)(blockIdx.x % KAON_RUN);
  if (sl >= run_slices(run)) return;
  const KaonItem it = slice_item(run, sl);
  const KaonTensor& T = D[it.tensor];
  const int cpl = (int)(((T.C >> 3) + 63) >> 6);
  constexpr int W = CODEC == KAON_MOM_INT8 ? 10 : 6;  // rows x chunks held per group
#define KAON_PNM_SS(N)                                                                 \
  case N: {                                                                            \
    constexpr int GR = W / N > 0 ? W / N : 1;                                          \
    pnm_ss_body<N, GR, CODEC>(T, it, ws, hp);                                          \
    break;                                                                             \
  }
  switch (cpl) {
    KAON_PNM_SS(1) KAON_PNM_SS(2) KAON_PNM_SS(3) KAON_PNM_SS(4)
  }
#undef KAON_PNM_SS
}

// =============================================================== MSAM norm="global"
// Sum of squares of the dequantized momentum (_global_mnorm, msam.py:191-199):
// each row in the 64-lane order into rs[r] (a 1-D tensor is one row); k_msq_fin
// adds the rows in the 64-lane order into the tensor's scalar word 2.
template <int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_msq(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, Ws ws) {
  const KaonItem run = items[blockIdx.x / KAON_RUN];
  const int sl = (int)(blockIdx.x % KAON_RUN);
  if (sl >= run_slices(run)) return;
  const KaonItem it = slice_item(run, sl);
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C;
  const int64_t nch = (C + 7) >> 3;
  const int cpl = (int)((nch + 63) >> 6);
  const bool vec = T.vec_rows != 0;
  const WaveRows wr = wave_rows(it);
  for (int64_t r = wr.rb; r < wr.re; ++r) {
    const float sc = CODEC == KAON_MOM_INT8 ? uniform_f(G(T.m_scale)[T.factored ? r : 0]) : 1.0f;
    float a = 0.0f;
    for (int k = 0; k < cpl; ++k) {
      const int64_t c = wr.lane + 64 * k;
      const int cnt = chunk_cnt(c, C);
      if (cnt <= 0) continue;
      const int64_t e0 = r * C + c * 8;
      uint32_t mq[8];
      ld_mom_at<CODEC>(T.m, e0, cnt, vec && cnt == 8, mq);
      // 4-bit: walk the blocks from the chunk's first element (32-bit: n < 2^32)
      uint32_t blk = 0u, boff = 0u;
      if (CODEC == KAON_MOM_4BIT) {
        blk = (uint32_t)e0 / (uint32_t)T.block4;
        boff = (uint32_t)e0 - blk * (uint32_t)T.block4;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i >= cnt) continue;
        float m;
        if (CODEC == KAON_MOM_INT8) {
          m = (float)(int8_t)(uint8_t)mq[i] * sc;
        } else if (CODEC == KAON_MOM_4BIT) {
          m = ((float)mq[i] - 8.0f) * G(T.m_scale)[blk];
          if (++boff == (uint32_t)T.block4) {
            boff = 0u;
            ++blk;
          }
        } else if (CODEC == KAON_MOM_BF16) {
          m = bf2f(mq[i]);
        } else {
          m = __uint_as_float(mq[i]);
        }
        a = a + m * m;
      }
    }
    const float s = wave_csum(a);
    if (wr.lane == 0) ws.rs(T)[r] = s;
  }
}

// k_msq on row class 0 (factored, 16-byte rows with C % 8 == 0, at most 4
// chunks per lane) with int8 or bf16 momenta: the same sums in the same order,
// with the chunks of GR rows loaded before their arithmetic and the int8 row
// scales read once per wave (one row per lane, then read across lanes).
template <int CPL, int GR, int CODEC>
__device__ __forceinline__ void msq_pf_body(const KaonTensor& T, const KaonItem& it, const Ws& ws) {
  constexpr bool I8 = CODEC == KAON_MOM_INT8;
  const uint32_t C = (uint32_t)T.C;
  const int nch = (int)(C >> 3);
  const WaveRows wr = wave_rows(it);
  const int nrows = (int)(wr.re - wr.rb);
  if (nrows <= 0) return;
  const KAON_G uint8_t* mb = (const KAON_G uint8_t*)G(T.m);
  const float sc_l = I8 ? G(T.m_scale)[lane_row(wr.rb, nrows, wr.lane)] : 1.0f;
  for (int j0 = 0; j0 < nrows; j0 += GR) {
    ku2 m8[GR][CPL];
    ku4 m16[GR][CPL];
#pragma unroll
    for (int j = 0; j < GR; ++j) {
      const uint32_t rowe = (uint32_t)(wr.rb + min(j0 + j, nrows - 1)) * C;
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        const uint32_t e0 = rowe + 8u * (uint32_t)min(wr.lane + 64 * k, nch - 1);
        if (I8) m8[j][k] = ld_stream<true>((const KAON_G ku2*)(mb + e0));
        else m16[j][k] = ld_stream<true>((const KAON_G ku4*)(mb + 2u * e0));
      }
    }
#pragma unroll
    for (int j = 0; j < GR; ++j) {
      const int jj = j0 + j;
      if (jj >= nrows) continue;
      const float sc = lane_val(sc_l, jj);
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        if (wr.lane + 64 * k >= nch) continue;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float m;
          if (I8) {
            const uint32_t w = i < 4 ? m8[j][k].x : m8[j][k].y;
            m = (float)(int8_t)(uint8_t)((w >> (8 * (i & 3))) & 0xFFu) * sc;
          } else {
            const uint32_t wv[4] = {m16[j][k].x, m16[j][k].y, m16[j][k].z, m16[j][k].w};
            m = (i & 1) ? __uint_as_float(wv[i >> 1] & 0xFFFF0000u) : __uint_as_float(wv[i >> 1] << 16);
          }
          a = a + m * m;
        }
      }
      const float s2 = wave_csum(a);
      if (wr.lane == 0) ws.rs(T)[wr.rb + jj] = s2;
    }
  }
}

template <int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_msq_pf(const KaonTensor* __restrict__ D,
                                                    const KaonItem* __restrict__ items, Ws ws) {
  const KaonItem run = items[blockIdx.x / KAON_RUN];
  const int sl = (int)(blockIdx.x % KAON_RUN);
  if (sl >= run_slices(run)) return;
  const KaonItem it = slice_item(run, sl);
  const KaonTensor& T = D[it.tensor];
  switch ((int)(((T.C >> 3) + 63) >> 6)) {
    case 1: msq_pf_body<1, CODEC == KAON_MOM_INT8 ? 16 : 8, CODEC>(T, it, ws); break;
    case 2: msq_pf_body<2, CODEC == KAON_MOM_INT8 ? 8 : 4, CODEC>(T, it, ws); break;
    case 3: msq_pf_body<3, CODEC == KAON_MOM_INT8 ? 5 : 3, CODEC>(T, it, ws); break;
    case 4: msq_pf_body<4, CODEC == KAON_MOM_INT8 ? 4 : 2, CODEC>(T, it, ws); break;
  }
}

__global__ __launch_bounds__(KAON_WG) void k_msq_fin(const KaonTensor* __restrict__ D, int32_t n_tensors, Ws ws) {
  const int t = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (t >= n_tensors) return;
  const KaonTensor& T = D[t];
  const int lane = threadIdx.x & 63;
  const int64_t R = T.n > 0 ? T.R : 0;
  const KAON_G float* rs = ws.rs(T);
  float a = 0.0f;
  for (int64_t c = lane; c * 8 < R; c += 64)
    for (int i = 0; i < 8; ++i)
      if (c * 8 + i < R) a = a + rs[c * 8 + i];
  const float ss = wave_csum(a);
  if (lane == 0) ws.scal(T)[2] = ss;
}

// =============================================================== KProdigy
// The two passes of KProdigy (src/kaon/kprodigy.py).  Pass 1 sees the gradient
// g' = GC(g), plus wd * p when the decay is coupled (_collect_grad, :342-349);
// pass 2 reads the GC'd gradient (:768-808).

// Clear the keep count and the 4-bit block absmax of every tensor.
__global__ __launch_bounds__(KAON_WG) void k_pd_zero(const KaonTensor* __restrict__ D, Ws ws, int codec) {
  const KaonTensor& T = D[blockIdx.x];
  if (threadIdx.x == 0) ((KAON_G uint32_t*)ws.scal(T))[1] = 0u;
  if (codec == KAON_MOM_4BIT) {
    const int64_t nb = nblocks4(T);
    for (int64_t b = threadIdx.x; b < nb; b += KAON_WG) ws.bamax(T)[b] = 0u;
  }
}

// Pass 1 over rows (_pass1_per_param, kprodigy.py:392-441; _update_momentum
// :723-741): the GC row means (kept for the later kernels), the first moment of
// d*g' in its codec -- fp32 m*beta1 + d(1-beta1) g'; bf16 storage rounds after
// mul_ and after add_, whose alpha torch rounds to bf16; int8 and 4-bit (a lerp
// toward d*g') leave the row / block absmax and the old scales, pass 2
// requantizes -- and the full second moment v*beta2 + d^2(1-beta2) g' g'.
template <int GT, int PT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_pd1(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C;
  const int64_t nch = (C + 7) >> 3;
  const int cpl = (int)((nch + 63) >> 6);
  const bool vec = T.vec_rows != 0;
  const bool gc = (hp.flags & KAON_F_GC) && T.factored;
  const bool coupled = (hp.flags & KAON_F_PD_COUPLED) != 0;
  const float tgb = rbf(hp.pd_tg);
  const int nsl = run_slices(it);
  BlkMax bm4;  // 4-bit blocks across chunks or rows
#pragma clang loop unroll(disable)
  for (int sl = 0; sl < nsl; ++sl) {
  const WaveRows wr = wave_rows(slice_item(it, sl));
  for (int64_t r = wr.rb; r < wr.re; ++r) {
    float mu = 0.0f;
    if (gc) {
      float a = 0.0f;
      for (int k = 0; k < cpl; ++k) {
        const int64_t c = wr.lane + 64 * k;
        const int cnt = chunk_cnt(c, C);
        if (cnt <= 0) continue;
        float x[8];
        ld8<GT>(T.g, r * C + c * 8, cnt, vec && cnt == 8, x);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i < cnt) a = a + x[i];
      }
      mu = round_to<GT>(wave_csum(a) / (float)C);
      if (wr.lane == 0) ws.mu(T)[r] = mu;
    }
    const int64_t sr = T.factored ? r : 0;
    const float oldsc = CODEC == KAON_MOM_INT8 ? uniform_f(G(T.m_scale)[sr]) : 1.0f;
    const bool dqf = fabsf(oldsc) < 0x1p120f;
    float amax = 0.0f;
    for (int k = 0; k < cpl; ++k) {
      const int64_t c = wr.lane + 64 * k;
      const int cnt = chunk_cnt(c, C);
      if (cnt <= 0) continue;
      const int64_t e0 = r * C + c * 8;
      const bool vv = vec && cnt == 8;
      float g[8];
      ld8<GT>(T.g, e0, cnt, vv, g);
      if (gc) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          float a0 = g[i] - mu, a1 = g[i + 1] - mu;
          round_pair<GT>(a0, a1);
          g[i] = a0;
          g[i + 1] = a1;
        }
      }
      if (coupled) {
        float p[8];
        ld8<PT>(T.p, e0, cnt, vv, p);
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = __fmaf_rn(hp.wdl, p[i], g[i]);
      }
      if (CODEC != KAON_MOM_NONE) {
        uint32_t mq[8];
        ld_mom_at<CODEC>(T.m, e0, cnt, vv, mq);
        if (CODEC == KAON_MOM_F32 || CODEC == KAON_MOM_BF16) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (CODEC == KAON_MOM_F32) {
              mq[i] = __float_as_uint(__fmaf_rn(hp.pd_tg, g[i], __uint_as_float(mq[i]) * hp.b1));
            } else {
              const float mb = rbf(bf2f(mq[i]) * hp.b1);
              mq[i] = f2bf(__fmaf_rn(tgb, rbf(g[i]), mb));
            }
          }
          st_mom_at<CODEC>(T.m, T.n, e0, cnt, vv, mq);
        } else {
          // 4-bit: the chunk's first block and offset (32-bit, n < 2^31), then walked
          uint32_t wblk = 0u, woff = 0u;
          if (CODEC == KAON_MOM_4BIT) {
            wblk = (uint32_t)e0 / (uint32_t)T.block4;
            woff = (uint32_t)e0 - wblk * (uint32_t)T.block4;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (i >= cnt) continue;
            if (CODEC == KAON_MOM_INT8) {
              const float mf = __fmaf_rn(hp.pd_tg, g[i], dq_int8(mq[i], oldsc, -128.0f * oldsc, dqf) * hp.b1);
              amax = fmaxf(amax, fabsf(mf));
            } else {
              const uint32_t blk = wblk;
              const bool blk_first = woff == 0u;
              if (++woff == (uint32_t)T.block4) {
                woff = 0u;
                ++wblk;
              }
              const float sc = G(T.m_scale)[blk];
              const float mf = klerp(((float)mq[i] - 8.0f) * sc, g[i] * hp.pd_d, hp.w1);
              bm4.add(ws.bamax(T), blk, fabsf(mf));
              if (blk_first) ws.boldsc(T, nblocks4(T))[blk] = sc;
            }
          }
        }
      }
      if (T.full_v) {
        float v[8];
        ld8<KAON_F32>(T.v, e0, cnt, vv, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __fmaf_rn(hp.pd_vval * g[i], g[i], v[i] * hp.b2);
        st8_f32(T.v, e0, cnt, vv, v);
      }
    }
    if (CODEC == KAON_MOM_INT8) {
      const float am = wave_max(amax);
      if (wr.lane == 0) {
        ws.ramax(T)[r] = __float_as_uint(am);
        ws.roldsc(T)[r] = oldsc;
      }
    }
  }
  }
  if (CODEC == KAON_MOM_4BIT) bm4.flush(ws.bamax(T));
}

// One element of a 16-bit or fp32 tensor, as fp32.
template <int DT>
__device__ __forceinline__ float ld1(const void* base, int64_t e) {
  return DT == KAON_F32 ? G((const float*)base)[e] : lp2f<DT>(G((const uint16_t*)base)[e]);
}

// Pass 1 for the tensors whose second moment is factored over their last two
// dims (factor_conv_as_matrix=False, kprodigy.py:286-288; update_factored_state
// and factored_inv_sqrt_factors, _factored.py:48-83, on the unreshaped weight):
// one thread per [fb_r, fb_c] block.  q = g'^2 (+eps1), g' = GC(g) with the row
// means k_pd1 stored (plus wd * p under the coupled decay); row[b, a] =
// lerp(row, mean_c q, 1-beta2), col[b, c] = lerp(col, mean_a q, 1-beta2), every
// sum sequential from +0.0f; then the block's factors for pass 2, c = 1 /
// sqrt(col) into the workspace's column words and r = 1 / sqrt(row / mean_a row)
// into its partial words.  Workgroup (t, y) takes tensor t's blocks y*256 + tid,
// stepping by gridDim.y * 256.
template <int GT, int PT>
__global__ __launch_bounds__(KAON_WG) void k_pd_bfac(const KaonTensor* __restrict__ D, Ws ws, KaonHyper hp) {
  const KaonTensor& T = D[blockIdx.x];
  if (T.fb_r <= 0 || T.n == 0) return;
  const int64_t Rb = T.fb_r, Cb = T.fb_c, bsz = Rb * Cb, nb = T.n / bsz;
  const bool gc = (hp.flags & KAON_F_GC) != 0;
  const bool coupled = (hp.flags & KAON_F_PD_COUPLED) != 0;
  const bool eps = (hp.flags & KAON_F_EPS) != 0;
  KAON_G float* cfb = ws.cf(T);
  KAON_G float* rfb = ws.part(T);
  KAON_G float* row = G(T.row);
  KAON_G float* col = G(T.col);
  for (int64_t b = (int64_t)blockIdx.y * KAON_WG + threadIdx.x; b < nb; b += (int64_t)gridDim.y * KAON_WG) {
    const int64_t e0 = b * bsz;
    const float mu = gc ? ws.mu(T)[e0 / T.C] : 0.0f;
    auto q = [&](int64_t e) {
      float x = ld1<GT>(T.g, e);
      if (gc) x = round_to<GT>(x - mu);
      if (coupled) x = __fmaf_rn(hp.wdl, ld1<PT>(T.p, e), x);
      float v = x * x;
      if (eps) v = v + hp.eps1;
      return v;
    };
    float rsum = 0.0f;
    for (int64_t a = 0; a < Rb; ++a) {
      float s = 0.0f;
      for (int64_t c = 0; c < Cb; ++c) s = s + q(e0 + a * Cb + c);
      const float nr = klerp(row[b * Rb + a], s / (float)Cb, hp.w2);
      row[b * Rb + a] = nr;
      rsum = rsum + nr;
    }
    for (int64_t c = 0; c < Cb; ++c) {
      float s = 0.0f;
      for (int64_t a = 0; a < Rb; ++a) s = s + q(e0 + a * Cb + c);
      const float nc = klerp(col[b * Cb + c], s / (float)Rb, hp.w2);
      col[b * Cb + c] = nc;
      cfb[b * Cb + c] = 1.0f / sqrtf(nc);
    }
    const float rm = rsum / (float)Rb;
    for (int64_t a = 0; a < Rb; ++a) rfb[b * Rb + a] = 1.0f / sqrtf(row[b * Rb + a] / rm);
  }
}

// Pass 1, D statistics: one wave per flat item of KAON_FLAT_ITEM sliced
// elements j (element j * slice_p): s_j = fma(alpha_s, g', s_j * beta3), and the
// item's sums of g' (p0 - p) and |s| in the 64-lane order (lane l adds chunks
// l, l+64, ... of 8 sliced elements), stored per item for k_pd_sfin.
template <int GT, int PT>
__global__ __launch_bounds__(KAON_WG) void k_pd_stats(const KaonTensor* __restrict__ D,
                                                      const KaonItem* __restrict__ items, int32_t n_items, Ws ws,
                                                      KaonHyper hp) {
  // sliced tensors (slice_p > 1): each wave stages one round of 512 sliced g
  // and p values here, loaded lane-interleaved (coalesced), then read back as
  // the lanes' 8-element chunks; only the wave itself touches its region
  __shared__ float stage[4][2][512];
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int64_t idx = (int64_t)blockIdx.x * 4 + w;
  if (idx >= n_items) return;
  const KaonItem it = items[idx];
  const KaonTensor& T = D[it.tensor];
  const int64_t sp = T.pd_slice, C = T.C, j0 = it.row0, len = it.nrows;
  const bool gc = (hp.flags & KAON_F_GC) && T.factored;
  const bool coupled = (hp.flags & KAON_F_PD_COUPLED) != 0;
  const KAON_G float* p0 = G(T.pd_p0);
  KAON_G float* sv = G(T.pd_s);
  float an = 0.0f, ad = 0.0f;
  const int64_t nch = (len + 7) >> 3;
  if (sp == 1) {
    // contiguous: 16-byte accesses for whole chunks (j0 and the chunks are 8-aligned)
    const bool vec = T.vec_flat != 0;
    for (int64_t c = lane; c < nch; c += 64) {
      const int64_t jj = c * 8, j = j0 + jj;
      const int cnt = (int)min<int64_t>(8, len - jj);
      const bool vv = vec && cnt == 8;
      float g[8], p[8], z[8], sc[8];
      ld8<GT>(T.g, j, cnt, vv, g);
      ld8<PT>(T.p, j, cnt, vv, p);
      ld8<KAON_F32>(T.pd_s, j, cnt, vv, sc);
      if (!T.pd_p0_scalar) ld8<KAON_F32>(T.pd_p0, j, cnt, vv, z);
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) z[i] = p0[0];
      // the GC row means of the chunk's elements: one 32-bit division per chunk, then a
      // walk along the row (n < 2^31)
      float mu[8];
      if (gc) {
        uint32_t r = (uint32_t)j / (uint32_t)C, c = (uint32_t)j - r * (uint32_t)C;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          mu[i] = i < cnt ? ws.mu(T)[r] : 0.0f;
          if (++c == (uint32_t)C) {
            c = 0u;
            ++r;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i >= cnt) continue;
        float gv = g[i];
        if (gc) gv = round_to<GT>(gv - mu[i]);
        if (coupled) gv = __fmaf_rn(hp.wdl, p[i], gv);
        an = an + gv * (z[i] - p[i]);
        sc[i] = __fmaf_rn(hp.pd_alpha_s, gv, sc[i] * hp.pd_beta3);
        ad = ad + fabsf(sc[i]);
      }
      st8_f32(T.pd_s, j, cnt, vv, sc);
    }
  } else {
    float* sg = stage[w][0];
    float* spv = stage[w][1];
    for (int64_t t = 0; 64 * t < nch; ++t) {
      // round t: chunks lane + 64 t, i.e. sliced elements 512 t .. 512 t + 511 of the item
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t jj = 512 * t + lane + 64 * u;
        float gv = 0.0f, pv = 0.0f;
        if (jj < len) {
          const int64_t e = (j0 + jj) * sp;
          gv = GT == KAON_F32 ? G((const float*)T.g)[e] : lp2f<GT>(G((const uint16_t*)T.g)[e]);
          pv = PT == KAON_F32 ? G((const float*)T.p)[e] : lp2f<PT>(G((const uint16_t*)T.p)[e]);
        }
        sg[lane + 64 * u] = gv;
        spv[lane + 64 * u] = pv;
      }
      // the wave's LDS writes before its reads of other lanes' values
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int64_t c = lane + 64 * t;
      // row of the chunk's first element, then walked by slice_p per element
      const uint32_t e_first = (uint32_t)((j0 + c * 8) * sp);
      uint32_t row = gc ? e_first / (uint32_t)C : 0u, col = gc ? e_first - row * (uint32_t)C : 0u;
      for (int i = 0; i < 8; ++i) {
        const int64_t jj = c * 8 + i;
        if (jj >= len) break;
        const int64_t j = j0 + jj;
        float gv = sg[8 * lane + i], pv = spv[8 * lane + i];
        if (gc) {
          gv = round_to<GT>(gv - ws.mu(T)[row]);
          col += (uint32_t)sp;
          while (col >= (uint32_t)C) {
            col -= (uint32_t)C;
            ++row;
          }
        }
        if (coupled) gv = __fmaf_rn(hp.wdl, pv, gv);
        const float pz = T.pd_p0_scalar ? p0[0] : p0[j];
        an = an + gv * (pz - pv);
        const float snew = __fmaf_rn(hp.pd_alpha_s, gv, sv[j] * hp.pd_beta3);
        sv[j] = snew;
        ad = ad + fabsf(snew);
      }
      // every lane's reads of this round before the next round's writes
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  const float num = wave_csum(an), den = wave_csum(ad);
  if (lane == 0) {
    const int64_t nfb = (T.pd_ns + KAON_FLAT_ITEM - 1) / KAON_FLAT_ITEM, blk = j0 / KAON_FLAT_ITEM;
    KAON_G float* bs = G(ws.base + T.ws_aux);
    bs[blk] = num;
    bs[nfb + blk] = den;
  }
}

// Each tensor's D statistics from its item sums, in the 64-lane order, into
// its scalar words 2 (num) and 3 (den).  One wave per tensor.
__global__ __launch_bounds__(KAON_WG) void k_pd_sfin(const KaonTensor* __restrict__ D, int32_t n_tensors, Ws ws) {
  const int t = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (t >= n_tensors) return;
  const KaonTensor& T = D[t];
  const int lane = threadIdx.x & 63;
  const int64_t nfb = (T.pd_ns + KAON_FLAT_ITEM - 1) / KAON_FLAT_ITEM;
  const KAON_G float* bs = G(ws.base + T.ws_aux);
  float a = 0.0f, b = 0.0f;
  for (int64_t c = lane; c * 8 < nfb; c += 64)
    for (int i = 0; i < 8; ++i) {
      const int64_t k = c * 8 + i;
      if (k < nfb) {
        a = a + bs[k];
        b = b + bs[nfb + k];
      }
    }
  const float sa = wave_csum(a), sb = wave_csum(b);
  if (lane == 0) {
    ws.scal(T)[2] = sa;
    ws.scal(T)[3] = sb;
  }
}

// Pass 2 (_update_one_param, kprodigy.py:768-808), phase 5 (cautious keep count)
// or 6 (apply): numerator = the momentum (float codecs as pass 1 stored it; int8 /
// 4-bit requantized here from the old codes with pass 1's absmax) or g; over
// max(sqrt(v), dn*eps), or times min(r c / dn, 1/(dn*eps)); times dlr; decoupled
// WD; cautious; write.  With KAON_F_GC_WRITE the apply also stores the
// centralized gradient over p.grad.
template <int PHASE, int PT, int GT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_pd2(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  __shared__ uint32_t keep_s[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const int64_t C = T.C, n = T.n;
  const int64_t nch = (C + 7) >> 3;
  const int cpl = (int)((nch + 63) >> 6);
  const bool vec_t = T.vec_rows != 0;
  const bool gc = (hp.flags & KAON_F_GC) && T.factored;
  const bool cautious = (hp.flags & KAON_F_CAUTIOUS) != 0;
  const bool decoupled_wd = (hp.flags & KAON_F_WD) != 0;
  const bool coupled = (hp.flags & KAON_F_PD_COUPLED) != 0;
  const bool lowp = PT == KAON_BF16;
  const bool factored = T.factored && !T.full_v;
  const int64_t B = CODEC == KAON_MOM_4BIT ? (int64_t)T.block4 : 1;
  const int64_t nb = CODEC == KAON_MOM_4BIT ? nblocks4(T) : 0;
  const WaveRows wr = wave_rows(it);
  double rden = 1.0;
  if (PHASE == 6 && cautious) {
    const uint32_t cnt = ((const KAON_G uint32_t*)ws.scal(T))[1];
    rden = rcp64(fmaxf((float)cnt / (float)n, 1e-8f));
  }
  uint32_t keep = 0;
  // the scales of the last 4-bit block visited: read once per run of its elements
  uint32_t c_blk = 0xFFFFFFFFu;
  float c_o = 1.0f, c_n = 1.0f;
  double c_r = 1.0;
  for (int64_t r = wr.rb; r < wr.re; ++r) {
    const float mu = gc ? uniform_f(ws.mu(T)[r]) : 0.0f;
    // block-factored tensors: r and c come per element (f below), the row factor is 1
    const float rf = factored ? (T.fb_r ? 1.0f : uniform_f(ws.rf(T)[r])) : 0.0f;
    float oldsc = 1.0f, newsc = 1.0f;
    double rnew = 1.0;
    if (CODEC == KAON_MOM_INT8) {
      oldsc = uniform_f(ws.roldsc(T)[r]);
      newsc = uniform_f(fmaxf(__uint_as_float(ws.ramax(T)[r]), 1e-12f) / 127.0f);
      rnew = rcp64(newsc);
    }
    const bool dqf = fabsf(oldsc) < 0x1p120f;
    for (int k = 0; k < cpl; ++k) {
      const int64_t c = wr.lane + 64 * k;
      const int cnt = chunk_cnt(c, C);
      if (cnt <= 0) continue;
      const int64_t j0 = c * 8;
      const int64_t e0 = r * C + j0;
      const bool vec = vec_t && cnt == 8;
      float g[8], p[8], f[8];
      uint32_t mq[8], pb[8];
      ld8<GT>(T.g, e0, cnt, vec, g);
      const bool need_p = PHASE == 6 || decoupled_wd || (coupled && (CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT));
      if (need_p) {
        if (PT != KAON_F32) {
          ld8_bits(T.p, e0, cnt, vec, pb);
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = lp2f<PT>(pb[i]);
        } else {
          ld8<KAON_F32>(T.p, e0, cnt, vec, p);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = 0.0f;
      }
      if (CODEC != KAON_MOM_NONE) ld_mom_at<CODEC>(T.m, e0, cnt, vec, mq);
      if (factored && T.fb_r) {
        // r c of each element's [fb_r, fb_c] block (n < 2^31: 32-bit indices)
        const uint32_t Rb = (uint32_t)T.fb_r, Cb = (uint32_t)T.fb_c, bsz = Rb * Cb;
        const KAON_G float* cfb = ws.cf(T);
        const KAON_G float* rfb = ws.part(T);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t e = (uint32_t)(e0 + min(i, cnt - 1));
          const uint32_t b = e / bsz, w = e - b * bsz, a = w / Cb, c = w - a * Cb;
          f[i] = rfb[b * Rb + a] * cfb[b * Cb + c];
        }
      } else if (factored) {
        ld8<KAON_F32>((const float*)ws.cf(T), j0, cnt, vec, f);
      } else {
        ld8<KAON_F32>(T.v, e0, cnt, vec, f);
      }
      uint32_t nz[8];
      if (PHASE == 6 && lowp && hp.bf16_method == KAON_SR) {
        if ((e0 & 7) == 0) noise8(hp.seed, hp.step, (uint32_t)T.tensor_id, 1u, e0, T.noise[1], cnt, nz);
        else
#pragma unroll
          for (int i = 0; i < 8; ++i) nz[i] = i < cnt ? noise1(hp.seed, hp.step, T.tensor_id, 1u, e0 + i, T.noise[1]) : 0u;
      }
      if (gc) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          float a0 = g[i] - mu, a1 = g[i + 1] - mu;
          round_pair<GT>(a0, a1);
          g[i] = a0;
          g[i + 1] = a1;
        }
      }
      uint32_t qout[8];
      float dout[8];
      // 4-bit: the chunk's first block and offset, walked element by element
      uint32_t wblk = 0u, woff = 0u;
      if (CODEC == KAON_MOM_4BIT) {
        wblk = (uint32_t)e0 / (uint32_t)B;
        woff = (uint32_t)e0 - wblk * (uint32_t)B;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qout[i] = mq[i];
        dout[i] = 0.0f;
        if (i >= cnt) continue;
        const float gq = coupled ? __fmaf_rn(hp.wdl, p[i], g[i]) : g[i];
        float numer;
        if (CODEC == KAON_MOM_NONE) {
          numer = g[i];
        } else if (CODEC == KAON_MOM_F32) {
          numer = __uint_as_float(mq[i]);
        } else if (CODEC == KAON_MOM_BF16) {
          numer = bf2f(mq[i]);
        } else if (CODEC == KAON_MOM_INT8) {
          const float mf = __fmaf_rn(hp.pd_tg, gq, dq_int8(mq[i], oldsc, -128.0f * oldsc, dqf) * hp.b1);
          float x = rintf(div_r64(mf, rnew));
          x = fminf(fmaxf(x, -127.0f), 127.0f);
          qout[i] = (uint32_t)(uint8_t)(int8_t)x;
          numer = x * newsc;
        } else {
          const int64_t blk = wblk;
          const bool blk_first = woff == 0u;
          if (++woff == (uint32_t)B) {
            woff = 0u;
            ++wblk;
          }
          if ((uint32_t)blk != c_blk) {  // the block's scales, once per run of its elements
            c_blk = (uint32_t)blk;
            c_o = ws.boldsc(T, nb)[blk];
            c_n = fmaxf(__uint_as_float(ws.bamax(T)[blk]), 1e-12f) / 7.0f;
            c_r = rcp64(c_n);
          }
          const float sco = c_o, scn = c_n;
          const float mf = klerp(((float)mq[i] - 8.0f) * sco, gq * hp.pd_d, hp.w1);
          float x = rintf(div_r64(mf, c_r));
          x = fminf(fmaxf(x, -7.0f), 7.0f);
          qout[i] = (uint32_t)((int)x + 8);
          numer = x * scn;
          if (PHASE == 6 && blk_first) G(T.m_scale)[blk] = scn;
        }
        const float u = factored ? numer * fminf((rf * f[i]) / hp.pd_dn, hp.pd_cap)
                                 : numer / fmaxf(sqrtf(f[i]), hp.pd_floor);
        float d = u * hp.pd_dlr;
        if (decoupled_wd) d = __fmaf_rn(hp.pd_wdl, p[i], d);
        const bool kp = d * g[i] > 0.0f;
        if (PHASE == 5) {
          keep += kp ? 1u : 0u;
          continue;
        }
        dout[i] = cautious ? div_r64(d * (kp ? 1.0f : 0.0f), rden) : d;
      }
      if (PHASE != 6) continue;
      if (gc && (hp.flags & KAON_F_GC_WRITE) && T.gc_write) {
        // the centralized gradient over p.grad (already rounded to the grad dtype)
        if (GT == KAON_F32) {
          st8_f32(const_cast<void*>(T.g), e0, cnt, vec, g);
        } else {
          uint32_t gb[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) gb[i] = f2lp<GT>(g[i]);
          st8_bits(const_cast<void*>(T.g), e0, cnt, vec, gb);
        }
      }
      if (CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT) st_mom_at<CODEC>(T.m, n, e0, cnt, vec, qout);
      if (PT == KAON_F32) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = p[i] - dout[i];
        st8_f32(T.p, e0, cnt, vec, o);
      } else {
        uint32_t o[8];
        if (hp.bf16_method == KAON_KAHAN) {
          uint32_t sh[8];
          ld8_bits(T.shift, e0, cnt, vec, sh);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            // shift -= lp(delta); p0 = p; p += shift; shift += p0 - p, in the
            // param dtype (_backend.py:90-94)
            const float s = round_to<PT>(lp2f<PT>(sh[i]) - round_to<PT>(dout[i]));
            const float p0 = p[i];
            const float p1 = round_to<PT>(p0 + s);
            o[i] = f2lp<PT>(p1);
            sh[i] = f2lp<PT>(s + round_to<PT>(p0 - p1));
          }
          st8_bits(T.shift, e0, cnt, vec, sh);
        } else if (hp.bf16_method == KAON_RN || PT == KAON_F16) {
          // fp16 params are written by RN under "stochastic_rounding" too: the
          // reference's SR write is bf16-only (_backend.py:95-98)
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = f2lp<PT>(p[i] - round_to<PT>(dout[i]));
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = sr_bf16(p[i] - dout[i], nz[i]);
        }
        st8_bits(T.p, e0, cnt, vec, o);
      }
    }
    if (PHASE == 6 && CODEC == KAON_MOM_INT8 && wr.lane == 0) G(T.m_scale)[T.factored ? r : 0] = newsc;
  }
  if (PHASE == 5 && cautious) {
    const uint32_t wsum = wave_sum_u32(keep);
    if (wr.lane == 0) keep_s[wr.w] = wsum;
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t tot = keep_s[0] + keep_s[1] + keep_s[2] + keep_s[3];
      if (tot) atomicAdd(ws.keep_ctr(T), tot);
    }
  }
}

// =============================================================== MSAM apply
// The centralized gradient written back over p.grad, as the reference's native
// path leaves it (centralize_grads_, _backend.py:147-177: g -= mean over the
// fan-in, in the grad dtype, for params of 2 dims or more): g = round(g - mu)
// with the row means phase 1 stored, for the tensors whose gc_write is set.
// One slice per workgroup.
template <int GT>
__global__ __launch_bounds__(KAON_WG) void k_gc_write(const KaonTensor* __restrict__ D,
                                                      const KaonItem* __restrict__ items, Ws ws) {
  const KaonItem run = items[blockIdx.x / KAON_RUN];
  const int sl = (int)(blockIdx.x % KAON_RUN);
  if (sl >= run_slices(run)) return;
  const KaonItem it = slice_item(run, sl);
  const KaonTensor& T = D[it.tensor];
  if (!T.factored || T.n == 0 || !T.gc_write) return;
  const int64_t C = T.C, nch = (C + 7) >> 3;
  const bool vec = T.vec_rows != 0;
  const WaveRows wr = wave_rows(it);
  for (int64_t r = wr.rb; r < wr.re; ++r) {
    const float mu = uniform_f(ws.mu(T)[r]);
    for (int64_t c = wr.lane; c < nch; c += 64) {
      const int cnt = chunk_cnt(c, C);
      const int64_t e0 = r * C + c * 8;
      const bool vv = vec && cnt == 8;
      float x[8];
      ld8<GT>(T.g, e0, cnt, vv, x);
      if (GT != KAON_F32) {
        uint32_t b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) b[i] = f2lp<GT>(x[i] - mu);
        st8_bits(const_cast<void*>(T.g), e0, cnt, vv, b);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = x[i] - mu;
        st8_f32(const_cast<void*>(T.g), e0, cnt, vv, x);
      }
    }
  }
}

template <int PT, int CODEC>
__global__ __launch_bounds__(KAON_WG) void k_msam(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, KaonHyper hp,
                                                  float factor, float bound, uint32_t sid, const float* wsb) {
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  if (wsb) {
    // norm="tensor" (msam.py:219-222): factor is sign * rho and bound is eps;
    // the tensor's own scale (sign * rho) / (||m|| + eps), evaluated as torch does
    // a python scalar over a tensor, reciprocal(||m|| + eps) * (sign * rho), with
    // ||m|| the square root of the sum kaon_momentum_sumsq left in scalar word 2
    const float nrm = sqrtf(G(wsb + T.ws_scal)[2]);
    factor = (1.0f / (nrm + bound)) * factor;
    bound = __builtin_inff();
  }
  const float nanfill = msam_nanfill(bound);
  // tensors hold < 2^32 elements: unsigned 32-bit element and row arithmetic
  const uint32_t e_begin = (uint32_t)it.row0, e_end = (uint32_t)it.row0 + (uint32_t)it.nrows;
  const bool vecT = T.vec_flat != 0;
  // the scale of element e is scale[e / span] (int8: span C per row, or the whole 1-D tensor;
  // 4-bit: the block); chunks start at multiples of 8, so a span that is a multiple of 8
  // gives one scale per chunk, and any other span is walked element by element
  const uint32_t span = CODEC == KAON_MOM_4BIT ? (uint32_t)T.block4
                        : (CODEC == KAON_MOM_INT8 && T.factored) ? (uint32_t)T.C : 0u;
  const bool span8 = span % 8u == 0u;
  const KAON_G float* msc = G(T.m_scale);
  for (uint32_t e0 = e_begin + 8u * threadIdx.x; e0 < e_end; e0 += 8u * KAON_WG) {
    const int cnt = (int)min(8u, e_end - e0);
    const bool vec = vecT && cnt == 8;
    uint32_t mq[8];
    ld_mom_raw<CODEC>(T, e0, cnt, vec, mq);
    float sc[8];
    if (CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT) {
      if (span == 0u) {
        const float s0 = msc[0];
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = s0;
      } else if (span8) {
        const float s0 = msc[e0 / span];
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = s0;
      } else {
        uint32_t r = e0 / span, c = e0 - r * span;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          sc[i] = i < cnt ? msc[r] : 0.0f;
          if (++c == span) {
            c = 0u;
            ++r;
          }
        }
      }
    }
    float ev[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float mold = 0.0f;
      if (i < cnt) {
        if (CODEC == KAON_MOM_INT8) mold = (float)(int8_t)(uint8_t)mq[i] * sc[i];
        else if (CODEC == KAON_MOM_4BIT) mold = ((float)mq[i] - 8.0f) * sc[i];
        else if (CODEC == KAON_MOM_BF16) mold = bf2f(mq[i]);
        else mold = __uint_as_float(mq[i]);
      }
      ev[i] = msam_e(mold * factor, bound, nanfill);
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

__global__ __launch_bounds__(KAON_WG) void k_copy(const ku4* __restrict__ src_, ku4* __restrict__ dst_, int64_t n16) {
  const KAON_G ku4* src = G(src_);
  KAON_G ku4* dst = G(dst_);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const ku4 a = ld_stream<true>(src + i), b = ld_stream<true>(src + i + stride);
    const ku4 c = ld_stream<true>(src + i + 2 * stride), d = ld_stream<true>(src + i + 3 * stride);
    st_stream(dst + i, a);
    st_stream(dst + i + stride, b);
    st_stream(dst + i + 2 * stride, c);
    st_stream(dst + i + 3 * stride, d);
  }
  for (; i < n16; i += stride) st_stream(dst + i, ld_stream<true>(src + i));
}

// ------------------------------------------------------------ dispatch tables

template <int OPT, int PHASE, int PT, int GT>
ElemFn elem_by_codec(int codec) {
  switch (codec) {
    case KAON_MOM_NONE: return k_elem<OPT, PHASE, PT, GT, KAON_MOM_NONE>;
    case KAON_MOM_F32: return k_elem<OPT, PHASE, PT, GT, KAON_MOM_F32>;
    case KAON_MOM_BF16: return k_elem<OPT, PHASE, PT, GT, KAON_MOM_BF16>;
    case KAON_MOM_INT8: return k_elem<OPT, PHASE, PT, GT, KAON_MOM_INT8>;
    case KAON_MOM_4BIT: return k_elem<OPT, PHASE, PT, GT, KAON_MOM_4BIT>;
  }
  return nullptr;
}

template <int OPT, int PHASE>
ElemFn elem_fn(int pt, int gt, int codec) {
  if (pt == KAON_BF16 && gt == KAON_BF16) return elem_by_codec<OPT, PHASE, KAON_BF16, KAON_BF16>(codec);
  if (pt == KAON_BF16 && gt == KAON_F32) return elem_by_codec<OPT, PHASE, KAON_BF16, KAON_F32>(codec);
  if (pt == KAON_F32 && gt == KAON_BF16) return elem_by_codec<OPT, PHASE, KAON_F32, KAON_BF16>(codec);
  if (pt == KAON_F32 && gt == KAON_F32) return elem_by_codec<OPT, PHASE, KAON_F32, KAON_F32>(codec);
  if constexpr (OPT == KAON_OPT_ADAKAON || OPT == KAON_OPT_LION || OPT == KAON_OPT_ADAMUON)
    if (pt == KAON_F16 && gt == KAON_F16) return elem_by_codec<OPT, PHASE, KAON_F16, KAON_F16>(codec);
  return nullptr;
}

int fast_flags(const KaonHyper& h) {
  int ff = 0;
  if (h.flags & KAON_F_GC) ff |= FF_GC;
  if (h.flags & KAON_F_CAUTIOUS) ff |= FF_CAUT;
  if (h.flags & KAON_F_WD) ff |= FF_WD;
  if (h.flags & KAON_F_NK_REMOVE) ff |= FF_NKR;
  if (h.flags & KAON_F_NK_CLIMB) ff |= FF_NKC;
  if ((h.flags & KAON_F_GC_WRITE) && (h.flags & KAON_F_GC)) ff |= FF_GCW;
  return ff;
}

// Phase 5 or 6 over the slices: the specialized kernel over elem_items[0,
// n_fast) when one exists for the configuration, the generic one over the rest.
template <int OPT, int PHASE>
int launch_elem(const KaonLaunch& L, Ws ws, const KaonHyper& h, int codec, hipStream_t st) {
  int32_t n_fast = L.n_fast;
  ElemFn ff = nullptr;
  if (n_fast > 0 && h.bf16_method == KAON_SR && h.p_dtype == KAON_BF16 && h.g_dtype == KAON_BF16)
    ff = fast_kernel(OPT, PHASE, codec, fast_flags(h));
  if (!ff) n_fast = 0;
  if (n_fast > 0) {
    hipLaunchKernelGGL(ff, dim3(n_fast), dim3(KAON_WG), 0, st, L.descs, L.elem_items, ws, h);
  }
  const int32_t rest = L.n_elem_items - n_fast;
  if (rest > 0) {
    ElemFn fg = elem_fn<OPT, PHASE>(h.p_dtype, h.g_dtype, codec);
    hipLaunchKernelGGL(fg, dim3(rest), dim3(KAON_WG), 0, st, L.descs, L.elem_items + n_fast, ws, h);
  }
  return check_launch(PHASE == 5 ? "kaon: keep-count launch" : "kaon: apply launch");
}

using StatsFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper, int);
// row classes (slices are sorted by class): 0-2 prefetching kernels, 3-5 rows
// of <= 4, 10, 24 chunks per lane in registers, 6 streamed rows; dynamic LDS
// holds one slice column partial
constexpr int kClassMaxC[KAON_ROW_CLASSES] = {4 * 512, 10 * 512, 24 * 512, 4 * 512, 10 * 512, 24 * 512, kSeg};

// eps: 0 none, 1 fused square (eps1 == 0 or >= 2^-100), 2 unfused (sq_chunk)
template <int GT>
StatsFn stats_fn_gt(int cls, int eps) {
  switch (cls) {
    case 0: return eps == 1 ? k_pf_stats<0, 1> : eps == 2 ? k_pf_stats<0, 2> : k_pf_stats<0, 0>;
    case 1: return eps == 1 ? k_pf_stats<1, 1> : eps == 2 ? k_pf_stats<1, 2> : k_pf_stats<1, 0>;
    case 2: return eps == 1 ? k_pf_stats_wide<1> : eps == 2 ? k_pf_stats_wide<2> : k_pf_stats_wide<0>;
    case 3: return k_stats<GT, 4>;
    case 4: return k_stats<GT, 10>;
    case 5: return k_stats<GT, 24>;
    case 6: return k_stats<GT, 0>;
  }
  return nullptr;
}
StatsFn stats_fn(int gt, int cls, int eps) {
  if (gt == KAON_F16) return cls >= 3 && cls != 5 ? stats_fn_gt<KAON_F16>(cls, eps) : nullptr;
  return gt == KAON_BF16 ? stats_fn_gt<KAON_BF16>(cls, eps) : stats_fn_gt<KAON_F32>(cls, eps);
}

using MsamFn = void (*)(const KaonTensor*, const KaonItem*, KaonHyper, float, float, uint32_t, const float*);
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

// Phase-1 launches, one per register class run (slices are sorted by class).
// KProdigy's coupled decay reads p beside g: the prefetching classes 0-2 then
// run on the register classes 3-5 of the same chunks per lane (the same order).
int launch_stats(const KaonLaunch& L, Ws ws, const KaonHyper& hp, int mode, hipStream_t st) {
  int32_t off = 0;
  const bool generic = mode == 0 && (hp.flags & KAON_F_PD_COUPLED) != 0;
  for (int cls = 0; cls < KAON_ROW_CLASSES; ++cls) {
    const int32_t cnt = L.row_runs[cls];
    if (cnt <= 0) continue;
    if (cls < 3 && hp.g_dtype != KAON_BF16) return fail("kaon: prefetching row class planned for non-bf16 grads");
    const int kcls = generic && cls < 3 ? cls + 3 : cls;
    const int eps = !(hp.flags & KAON_F_EPS) ? 0 : (hp.eps1 == 0.0f || hp.eps1 >= 0x1p-100f) ? 1 : 2;
    StatsFn fn = stats_fn(hp.g_dtype, kcls, eps);
    if (!fn) return fail("kaon: no row-statistics kernel for this grad dtype and row class");
    const size_t lds = (mode == 0 && kcls >= 3) ? sizeof(float) * (size_t)kClassMaxC[kcls] : 0;
    hipLaunchKernelGGL(fn, dim3(cnt), dim3(KAON_WG), lds, st, L.descs, L.row_items + off, ws, hp, mode);
    off += cnt;
  }
  if (off != L.n_row_items) return fail("kaon: slice class runs do not add up to n_row_items");
  return check_launch("kaon: k_stats launch");
}

using MuonMomFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper);
template <int GT>
MuonMomFn muon_mom_gt(int codec) {
  switch (codec) {
    case KAON_MOM_NONE: return k_muon_mom<GT, KAON_MOM_NONE>;
    case KAON_MOM_F32: return k_muon_mom<GT, KAON_MOM_F32>;
    case KAON_MOM_BF16: return k_muon_mom<GT, KAON_MOM_BF16>;
    case KAON_MOM_INT8: return k_muon_mom<GT, KAON_MOM_INT8>;
    case KAON_MOM_4BIT: return k_muon_mom<GT, KAON_MOM_4BIT>;
  }
  return nullptr;
}

using PnmFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper);
template <int PHASE, int PT, int GT>
PnmFn pnm_by_codec(int codec) {
  switch (codec) {
    case KAON_MOM_F32: return k_pnm<PHASE, PT, GT, KAON_MOM_F32>;
    case KAON_MOM_BF16: return k_pnm<PHASE, PT, GT, KAON_MOM_BF16>;
    case KAON_MOM_INT8: return k_pnm<PHASE, PT, GT, KAON_MOM_INT8>;
    case KAON_MOM_4BIT: return k_pnm<PHASE, PT, GT, KAON_MOM_4BIT>;
  }
  return nullptr;
}
template <int PHASE>
PnmFn pnm_fn(int pt, int gt, int codec) {
  if (pt == KAON_BF16 && gt == KAON_BF16) return pnm_by_codec<PHASE, KAON_BF16, KAON_BF16>(codec);
  if (pt == KAON_BF16 && gt == KAON_F32) return pnm_by_codec<PHASE, KAON_BF16, KAON_F32>(codec);
  if (pt == KAON_F32 && gt == KAON_BF16) return pnm_by_codec<PHASE, KAON_F32, KAON_BF16>(codec);
  if (pt == KAON_F32 && gt == KAON_F32) return pnm_by_codec<PHASE, KAON_F32, KAON_F32>(codec);
  if (pt == KAON_F16 && gt == KAON_F16) return pnm_by_codec<PHASE, KAON_F16, KAON_F16>(codec);
  return nullptr;
}

using PdFn = void (*)(const KaonTensor*, const KaonItem*, Ws, KaonHyper);
using PdStatsFn = void (*)(const KaonTensor*, const KaonItem*, int32_t, Ws, KaonHyper);
template <int GT, int PT>
PdFn pd1_by_codec(int codec) {
  switch (codec) {
    case KAON_MOM_NONE: return k_pd1<GT, PT, KAON_MOM_NONE>;
    case KAON_MOM_F32: return k_pd1<GT, PT, KAON_MOM_F32>;
    case KAON_MOM_BF16: return k_pd1<GT, PT, KAON_MOM_BF16>;
    case KAON_MOM_INT8: return k_pd1<GT, PT, KAON_MOM_INT8>;
    case KAON_MOM_4BIT: return k_pd1<GT, PT, KAON_MOM_4BIT>;
  }
  return nullptr;
}
PdFn pd1_fn(int pt, int gt, int codec) {
  if (gt == KAON_F16 && pt == KAON_F16) return pd1_by_codec<KAON_F16, KAON_F16>(codec);
  if (gt == KAON_BF16 && pt == KAON_BF16) return pd1_by_codec<KAON_BF16, KAON_BF16>(codec);
  if (gt == KAON_BF16 && pt == KAON_F32) return pd1_by_codec<KAON_BF16, KAON_F32>(codec);
  if (gt == KAON_F32 && pt == KAON_BF16) return pd1_by_codec<KAON_F32, KAON_BF16>(codec);
  if (gt == KAON_F32 && pt == KAON_F32) return pd1_by_codec<KAON_F32, KAON_F32>(codec);
  return nullptr;
}
using PdBfacFn = void (*)(const KaonTensor*, Ws, KaonHyper);
PdBfacFn pd_bfac_fn(int pt, int gt) {
  if (gt == KAON_F16 && pt == KAON_F16) return k_pd_bfac<KAON_F16, KAON_F16>;
  if (gt == KAON_BF16 && pt == KAON_BF16) return k_pd_bfac<KAON_BF16, KAON_BF16>;
  if (gt == KAON_BF16 && pt == KAON_F32) return k_pd_bfac<KAON_BF16, KAON_F32>;
  if (gt == KAON_F32 && pt == KAON_BF16) return k_pd_bfac<KAON_F32, KAON_BF16>;
  if (gt == KAON_F32 && pt == KAON_F32) return k_pd_bfac<KAON_F32, KAON_F32>;
  return nullptr;
}
PdStatsFn pd_stats_fn(int pt, int gt) {
  if (gt == KAON_F16 && pt == KAON_F16) return k_pd_stats<KAON_F16, KAON_F16>;
  if (gt == KAON_BF16 && pt == KAON_BF16) return k_pd_stats<KAON_BF16, KAON_BF16>;
  if (gt == KAON_BF16 && pt == KAON_F32) return k_pd_stats<KAON_BF16, KAON_F32>;
  if (gt == KAON_F32 && pt == KAON_BF16) return k_pd_stats<KAON_F32, KAON_BF16>;
  if (gt == KAON_F32 && pt == KAON_F32) return k_pd_stats<KAON_F32, KAON_F32>;
  return nullptr;
}
template <int PHASE, int PT, int GT>
PdFn pd2_by_codec(int codec) {
  switch (codec) {
    case KAON_MOM_NONE: return k_pd2<PHASE, PT, GT, KAON_MOM_NONE>;
    case KAON_MOM_F32: return k_pd2<PHASE, PT, GT, KAON_MOM_F32>;
    case KAON_MOM_BF16: return k_pd2<PHASE, PT, GT, KAON_MOM_BF16>;
    case KAON_MOM_INT8: return k_pd2<PHASE, PT, GT, KAON_MOM_INT8>;
    case KAON_MOM_4BIT: return k_pd2<PHASE, PT, GT, KAON_MOM_4BIT>;
  }
  return nullptr;
}
template <int PHASE>
PdFn pd2_fn(int pt, int gt, int codec) {
  if (pt == KAON_F16 && gt == KAON_F16) return pd2_by_codec<PHASE, KAON_F16, KAON_F16>(codec);
  if (pt == KAON_BF16 && gt == KAON_BF16) return pd2_by_codec<PHASE, KAON_BF16, KAON_BF16>(codec);
  if (pt == KAON_BF16 && gt == KAON_F32) return pd2_by_codec<PHASE, KAON_BF16, KAON_F32>(codec);
  if (pt == KAON_F32 && gt == KAON_BF16) return pd2_by_codec<PHASE, KAON_F32, KAON_BF16>(codec);
  if (pt == KAON_F32 && gt == KAON_F32) return pd2_by_codec<PHASE, KAON_F32, KAON_F32>(codec);
  return nullptr;
}

// The second stream of a torch-order Adakaon step (the long tensors' clip
// chains), one per device, created on first use with default priority and
// non-blocking (no implicit order with the legacy default stream), with the
// fork and join events.  The mutex is held while a step enqueues its fork and
// join, so steps issued from several host threads do not interleave their
// records of the shared events.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  std::mutex mu;
};
constexpr int kSideDevices = 64;
SideStream g_side[kSideDevices];
std::mutex g_side_mu;

int side_stream(SideStream** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail("kaon: hipGetDevice", e);
  if (dev < 0 || dev >= kSideDevices) return fail("kaon: device index out of range for the side stream");
  std::lock_guard<std::mutex> lock(g_side_mu);
  SideStream& ss = g_side[dev];
  if (!ss.s) {
    // all three or none: a failed call leaves nothing behind for the next to trip on
    hipEvent_t fork = nullptr, join = nullptr;
    hipStream_t st = nullptr;
    if ((e = hipEventCreateWithFlags(&fork, hipEventDisableTiming)) == hipSuccess &&
        (e = hipEventCreateWithFlags(&join, hipEventDisableTiming)) == hipSuccess &&
        (e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) == hipSuccess) {
      ss.fork = fork;
      ss.join = join;
      ss.s = st;
    } else {
      if (join) (void)hipEventDestroy(join);
      if (fork) (void)hipEventDestroy(fork);
      return fail("kaon: side stream", e);
    }
  }
  *out = &ss;
  return 0;
}

// half_ok: the entry point steps fp16 params (Adakaon, Lion, AdaMuon, AdaPNM, KProdigy
// and the gradient write-back); their grads are fp16 too and no Nekaon / MSAM perturbation
// rides along (the reference's add_stochastic_ has no fp16 path,
// _stochastic_rounding.py:55-68).
int validate(const KaonLaunch* L, const KaonHyper* hp, const char* who, bool half_ok = false) {
  if (!L || !hp) return fail(who);
  if (hp->p_dtype != KAON_F32 && hp->p_dtype != KAON_BF16 && hp->p_dtype != KAON_F16)
    return fail("kaon: bad p_dtype");
  if (hp->g_dtype != KAON_F32 && hp->g_dtype != KAON_BF16 && hp->g_dtype != KAON_F16)
    return fail("kaon: bad g_dtype");
  if (hp->p_dtype == KAON_F16 || hp->g_dtype == KAON_F16) {
    if (!half_ok)
      return fail((std::string(who) + ": fp16 params step in Adakaon, Lion, AdaMuon, AdaPNM and KProdigy plans only").c_str());
    if (hp->p_dtype != KAON_F16 || hp->g_dtype != KAON_F16) return fail("kaon: fp16 params take fp16 grads");
    if (hp->flags & (KAON_F_NK_REMOVE | KAON_F_NK_CLIMB))
      return fail("kaon: the Nekaon / MSAM perturbation has no fp16 write (add_stochastic_ is bf16 / fp32 only)");
  }
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
  int rc = validate(L, hp, "kaon_adakaon_phases: null argument", true);
  if (rc) return rc;
  if (L->n_tensors <= 0 || L->n_row_items <= 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  const bool mom = (h.flags & KAON_F_MOMENTUM) && h.codec != KAON_MOM_NONE;
  const int codec = mom ? h.codec : KAON_MOM_NONE;
  if (!mom) h.flags &= ~(KAON_F_MOMENTUM | KAON_F_NK_REMOVE | KAON_F_NK_CLIMB);
  h.codec = codec;
  const bool quant = codec == KAON_MOM_INT8 || codec == KAON_MOM_4BIT;
  // phases 5 and 6 over a launch's elem items (or a sub-range of them)
  auto elem_phases = [&](const KaonLaunch& l) {
    int r = 0;
    if ((mask & (1u << 5)) && ((h.flags & KAON_F_CAUTIOUS) || quant) &&
        (r = launch_elem<KAON_OPT_ADAKAON, 5>(l, ws, h, codec, st)))
      return r;
    if ((mask & (1u << 6)) && (r = launch_elem<KAON_OPT_ADAKAON, 6>(l, ws, h, codec, st))) return r;
    return 0;
  };
  // the long-chain split as the planner left it (a caller that lowers n_fast
  // below n_long_fast, to send items to the generic kernel, gets one stream)
  const bool split_ok = L->n_long > 0 && L->n_long < L->n_tensors && L->n_long_fast >= 0 &&
                        L->n_long_fast <= L->n_fast && L->n_long_rest >= 0 &&
                        L->n_long_rest <= L->n_elem_items - L->n_fast;
  if ((h.flags & KAON_F_TORCH_ORDER) && split_ok && (mask & 0x68u) == 0x68u) {
    // The torch-order clip norm is n / 8 dependent fmas per tensor; the long
    // tensors' chains run on the side stream while the launch stream does the
    // other tensors' clip, keep count and apply, then theirs.  Each tensor's
    // kernels and their order are those of the one-stream step.
    int e = torch_phases(*L, ws, h, mask & 0x06u, 0, st);
    if (e) return fail("kaon: torch-order sum launch", (hipError_t)e);
    SideStream* ss = nullptr;
    if ((rc = side_stream(&ss))) return rc;
    // the elem items of the long tensors (leading in both parts) and of the others
    KaonLaunch lf = *L, lr = *L, sf = *L, sr = *L;
    lf.n_fast = lf.n_elem_items = L->n_long_fast;
    lr.elem_items = L->elem_items + L->n_fast;
    lr.n_fast = 0;
    lr.n_elem_items = L->n_long_rest;
    sf.elem_items = L->elem_items + L->n_long_fast;
    sf.n_fast = sf.n_elem_items = L->n_fast - L->n_long_fast;
    sr.elem_items = L->elem_items + L->n_fast + L->n_long_rest;
    sr.n_fast = 0;
    sr.n_elem_items = L->n_elem_items - L->n_fast - L->n_long_rest;
    std::lock_guard<std::mutex> lock(ss->mu);
    hipError_t he;
    if ((he = hipEventRecord(ss->fork, st)) != hipSuccess) return fail("kaon: side-stream fork", he);
    if ((he = hipStreamWaitEvent(ss->s, ss->fork, 0)) != hipSuccess) return fail("kaon: side-stream fork", he);
    if ((e = torch_clip(*L, ws, h, 0, L->n_long, ss->s))) return fail("kaon: torch-order clip launch", (hipError_t)e);
    if ((he = hipEventRecord(ss->join, ss->s)) != hipSuccess) return fail("kaon: side-stream join", he);
    if ((e = torch_clip(*L, ws, h, L->n_long, L->n_tensors, st)))
      return fail("kaon: torch-order clip launch", (hipError_t)e);
    if ((rc = elem_phases(sf)) || (rc = elem_phases(sr))) return rc;
    if ((he = hipStreamWaitEvent(st, ss->join, 0)) != hipSuccess) return fail("kaon: side-stream join", he);
    if ((rc = elem_phases(lf)) || (rc = elem_phases(lr))) return rc;
    return 0;
  }
  if (h.flags & KAON_F_TORCH_ORDER) {
    // the GC / row / column / row-factor means and the clip norm in torch CPU's order
    const int e = torch_phases(*L, ws, h, mask & 0x1Eu, 0, st);
    if (e) return fail("kaon: torch-order sum launch", (hipError_t)e);
  } else {
    if (mask & (1u << 1)) {
      if ((rc = launch_stats(*L, ws, h, 0, st))) return rc;
    }
    if ((mask & (1u << 2)) && L->n_fin_items > 0) {
      hipLaunchKernelGGL(k_fin, dim3(L->n_fin_items), dim3(KAON_WG), 0, st, L->descs, L->fin_items, ws, h);
      if ((rc = check_launch("kaon: k_fin launch"))) return rc;
    }
    // phase 3 (the clip's sum of squares) is folded into phases 1 and 2
    if (mask & (1u << 4)) {
      hipLaunchKernelGGL(k_clipdiv, dim3((L->n_tensors + 3) / 4), dim3(KAON_WG), 0, st, L->descs, L->n_tensors, ws,
                         h);
      if ((rc = check_launch("kaon: k_clipdiv launch"))) return rc;
    }
  }
  return elem_phases(*L);
}

int kaon_adakaon_step(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  return kaon_adakaon_phases(L, hp, 0x7Eu, stream);
}

int kaon_adamuon_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream) {
  int rc = validate(L, hp, "kaon_adamuon_phases: null argument", true);
  if (rc) return rc;
  if (hp->flags & KAON_F_TORCH_ORDER)
    return fail("kaon_adamuon_step: torch-order sums are built for the Adakaon (Nekaon, MSAM) and Lion steps");
  if (L->n_tensors <= 0 || L->n_row_items <= 0) return 0;
  if (L->n_ns_rect <= 0) return fail("kaon_adamuon: the launch was not planned for AdaMuon (no Newton-Schulz tiles)");
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  const bool mom = (h.flags & KAON_F_MOMENTUM) && h.codec != KAON_MOM_NONE;
  const int codec = mom ? h.codec : KAON_MOM_NONE;
  if (!mom) h.flags &= ~KAON_F_MOMENTUM;
  h.flags &= ~(KAON_F_NK_REMOVE | KAON_F_NK_CLIMB | KAON_F_SRC_O);
  h.codec = codec;
  // 8: momentum of the raw grad, its norm
  if (mask & (1u << 8)) {
    if (codec == KAON_MOM_4BIT) {
      hipLaunchKernelGGL(k_muon_zero, dim3(L->n_tensors), dim3(KAON_WG), 0, st, L->descs, L->n_tensors, ws);
      if ((rc = check_launch("kaon: AdaMuon zero launch"))) return rc;
    }
    MuonMomFn fm = h.g_dtype == KAON_BF16  ? muon_mom_gt<KAON_BF16>(codec)
                   : h.g_dtype == KAON_F16 ? muon_mom_gt<KAON_F16>(codec)
                                           : muon_mom_gt<KAON_F32>(codec);
    hipLaunchKernelGGL(fm, dim3(L->n_row_items), dim3(KAON_WG), 0, st, L->descs, L->row_items, ws, h);
    hipLaunchKernelGGL(k_muon_norm, dim3((L->n_tensors + 3) / 4), dim3(KAON_WG), 0, st, L->descs, L->n_tensors, ws);
    if ((rc = check_launch("kaon: AdaMuon momentum launch"))) return rc;
  }
  // 9: Newton-Schulz -> O
  if (mask & (1u << 9)) {
    if ((rc = kaon_ns_run(*L, h.ns_steps, st))) return rc;
  }
  // 1-4 on O: bf16 source, no GC (it applies to the grad), nothing of the
  // momentum codec (its block absmax is already accumulated)
  KaonHyper ho = h;
  ho.flags = (h.flags & ~KAON_F_GC) | KAON_F_SRC_O;
  ho.g_dtype = KAON_BF16;
  ho.codec = KAON_MOM_NONE;
  if (mask & (1u << 1)) {
    if ((rc = launch_stats(*L, ws, ho, 0, st))) return rc;
  }
  if ((mask & (1u << 2)) && L->n_fin_items > 0) {
    hipLaunchKernelGGL(k_fin, dim3(L->n_fin_items), dim3(KAON_WG), 0, st, L->descs, L->fin_items, ws, ho);
    if ((rc = check_launch("kaon: k_fin launch"))) return rc;
  }
  // phase 3 (the clip's sum of squares) is folded into phases 1 and 2
  if (mask & (1u << 4)) {
    hipLaunchKernelGGL(k_clipdiv, dim3((L->n_tensors + 3) / 4), dim3(KAON_WG), 0, st, L->descs, L->n_tensors, ws, ho);
    if ((rc = check_launch("kaon: k_clipdiv launch"))) return rc;
  }
  // 5-6: cautious count against the grad; requant, write
  if ((mask & (1u << 5)) && (h.flags & KAON_F_CAUTIOUS)) {
    if ((rc = launch_elem<KAON_OPT_ADAMUON, 5>(*L, ws, h, codec, st))) return rc;
  }
  if (mask & (1u << 6)) {
    if ((rc = launch_elem<KAON_OPT_ADAMUON, 6>(*L, ws, h, codec, st))) return rc;
  }
  return 0;
}

int kaon_adamuon_step(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  return kaon_adamuon_phases(L, hp, 0x37Eu, stream);
}

int kaon_adapnm_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream) {
  int rc = validate(L, hp, "kaon_adapnm_phases: null argument", true);
  if (rc) return rc;
  if (hp->flags & KAON_F_TORCH_ORDER)
    return fail("kaon_adapnm_step: torch-order sums are built for the Adakaon (Nekaon, MSAM) and Lion steps");
  if (L->n_tensors <= 0 || L->n_row_items <= 0) return 0;
  if (hp->codec == KAON_MOM_NONE) return fail("kaon_adapnm_step: AdaPNM keeps two momentum buffers; pass their codec");
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  h.flags |= KAON_F_PNM | KAON_F_MOMENTUM;
  h.flags &= ~(KAON_F_NK_REMOVE | KAON_F_NK_CLIMB | KAON_F_SRC_O);
  PnmFn f3 = pnm_fn<3>(h.p_dtype, h.g_dtype, h.codec);
  PnmFn f5 = pnm_fn<5>(h.p_dtype, h.g_dtype, h.codec);
  PnmFn f6 = pnm_fn<6>(h.p_dtype, h.g_dtype, h.codec);
  if (!f3 || !f5 || !f6) return fail("kaon_adapnm_step: unsupported dtype / codec combination");
  if (mask & (1u << 1)) {
    if ((rc = launch_stats(*L, ws, h, 0, st))) return rc;
  }
  if ((mask & (1u << 2)) && L->n_fin_items > 0) {
    hipLaunchKernelGGL(k_fin, dim3(L->n_fin_items), dim3(KAON_WG), 0, st, L->descs, L->fin_items, ws, h);
    if ((rc = check_launch("kaon: k_fin launch"))) return rc;
  }
  if (mask & (1u << 3)) {
    // row class 0 (the leading row items) with int8 / bf16 momenta: the prefetching kernel
    // (on the longer rows of class 1 it measured slower than the generic one with int8)
    PnmFn f3p = h.g_dtype != KAON_BF16 ? nullptr
                : h.codec == KAON_MOM_INT8 ? (PnmFn)k_pnm_ss<KAON_MOM_INT8>
                : h.codec == KAON_MOM_BF16 ? (PnmFn)k_pnm_ss<KAON_MOM_BF16> : nullptr;
    const int32_t n0 = f3p ? L->row_runs[0] : 0;
    if (n0 > 0)
      hipLaunchKernelGGL(f3p, dim3(n0 * KAON_RUN), dim3(KAON_WG), 0, st, L->descs, L->row_items, ws, h);
    if (L->n_row_items > n0)
      hipLaunchKernelGGL(f3, dim3((L->n_row_items - n0) * KAON_RUN), dim3(KAON_WG), 0, st, L->descs,
                         L->row_items + n0, ws, h);
    if ((rc = check_launch("kaon: AdaPNM clip-sum launch"))) return rc;
  }
  if (mask & (1u << 4)) {
    hipLaunchKernelGGL(k_clipdiv, dim3((L->n_tensors + 3) / 4), dim3(KAON_WG), 0, st, L->descs, L->n_tensors, ws, h);
    if ((rc = check_launch("kaon: k_clipdiv launch"))) return rc;
  }
  // phases 5 and 6: the specialized kernel over the fast slices when one exists
  // for the configuration, the generic one over the rest
  const bool fast_cfg = L->n_fast > 0 && h.bf16_method == KAON_SR && h.p_dtype == KAON_BF16 &&
                        h.g_dtype == KAON_BF16;
  auto launch_pnm = [&](ElemFn ff, PnmFn fg, const char* what) {
    const int32_t n_fast = ff ? L->n_fast : 0;
    if (n_fast > 0)
      hipLaunchKernelGGL(ff, dim3(n_fast), dim3(KAON_WG), 0, st, L->descs, L->elem_items, ws, h);
    if (L->n_elem_items > n_fast)
      hipLaunchKernelGGL(fg, dim3(L->n_elem_items - n_fast), dim3(KAON_WG), 0, st, L->descs,
                         L->elem_items + n_fast, ws, h);
    return check_launch(what);
  };
  if ((mask & (1u << 5)) && (h.flags & KAON_F_CAUTIOUS) && L->n_elem_items > 0) {
    ElemFn ff = fast_cfg ? fast_kernel(KAON_OPT_ADAPNM, 5, h.codec, fast_flags(h)) : nullptr;
    if ((rc = launch_pnm(ff, f5, "kaon: AdaPNM keep-count launch"))) return rc;
  }
  if ((mask & (1u << 6)) && L->n_elem_items > 0) {
    ElemFn ff = fast_cfg ? fast_kernel(KAON_OPT_ADAPNM, 6, h.codec, fast_flags(h)) : nullptr;
    if ((rc = launch_pnm(ff, f6, "kaon: AdaPNM apply launch"))) return rc;
  }
  return 0;
}

int kaon_adapnm_step(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  return kaon_adapnm_phases(L, hp, 0x7Eu, stream);
}

int kaon_momentum_sumsq(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  int rc = validate(L, hp, "kaon_momentum_sumsq: null argument");
  if (rc) return rc;
  if (L->n_tensors <= 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  if (hp->flags & KAON_F_TORCH_ORDER) {
    if (hp->codec == KAON_MOM_NONE) return fail("kaon_momentum_sumsq: needs a momentum codec");
    const int e = torch_momentum_sumsq(*L, ws, hp->codec, st);
    if (e) return fail("kaon: torch-order momentum sum launch", (hipError_t)e);
    return 0;
  }
  using MsqFn = void (*)(const KaonTensor*, const KaonItem*, Ws);
  MsqFn f = nullptr;
  switch (hp->codec) {
    case KAON_MOM_F32: f = k_msq<KAON_MOM_F32>; break;
    case KAON_MOM_BF16: f = k_msq<KAON_MOM_BF16>; break;
    case KAON_MOM_INT8: f = k_msq<KAON_MOM_INT8>; break;
    case KAON_MOM_4BIT: f = k_msq<KAON_MOM_4BIT>; break;
  }
  if (!f) return fail("kaon_momentum_sumsq: needs a momentum codec");
  // row class 0 (the leading row items) with int8 / bf16 momenta: the prefetching form
  MsqFn fp = hp->codec == KAON_MOM_INT8 ? k_msq_pf<KAON_MOM_INT8>
             : hp->codec == KAON_MOM_BF16 ? k_msq_pf<KAON_MOM_BF16> : nullptr;
  const int32_t n0 = fp ? L->row_runs[0] : 0;
  if (n0 > 0) hipLaunchKernelGGL(fp, dim3(n0 * KAON_RUN), dim3(KAON_WG), 0, st, L->descs, L->row_items, ws);
  if (L->n_row_items > n0)
    hipLaunchKernelGGL(f, dim3((L->n_row_items - n0) * KAON_RUN), dim3(KAON_WG), 0, st, L->descs,
                       L->row_items + n0, ws);
  hipLaunchKernelGGL(k_msq_fin, dim3((L->n_tensors + 3) / 4), dim3(KAON_WG), 0, st, L->descs, L->n_tensors, ws);
  return check_launch("kaon: momentum sum-of-squares launch");
}

int kaon_kprodigy_pass1(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  int rc = validate(L, hp, "kaon_kprodigy_pass1: null argument", true);
  if (rc) return rc;
  if (hp->flags & KAON_F_TORCH_ORDER)
    return fail("kaon_kprodigy_pass1: torch-order sums are built for the Adakaon (Nekaon, MSAM) and Lion steps");
  if (L->n_tensors <= 0 || L->n_row_items <= 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  const bool mom = (h.flags & KAON_F_MOMENTUM) && h.codec != KAON_MOM_NONE;
  const int codec = mom ? h.codec : KAON_MOM_NONE;
  h.codec = codec;
  h.flags &= ~(KAON_F_NK_REMOVE | KAON_F_NK_CLIMB | KAON_F_SRC_O | KAON_F_PNM);
  PdFn f1 = pd1_fn(h.p_dtype, h.g_dtype, codec);
  PdStatsFn fs = pd_stats_fn(h.p_dtype, h.g_dtype);
  if (!f1 || !fs) return fail("kaon_kprodigy_pass1: unsupported dtype / codec combination");
  hipLaunchKernelGGL(k_pd_zero, dim3(L->n_tensors), dim3(KAON_WG), 0, st, L->descs, ws, codec);
  if ((rc = check_launch("kaon: KProdigy zero launch"))) return rc;
  // the factored row/col EMAs (tensors with a per-element v return at once)
  if ((rc = launch_stats(*L, ws, h, 0, st))) return rc;
  if (L->n_fin_items > 0) {
    hipLaunchKernelGGL(k_fin, dim3(L->n_fin_items), dim3(KAON_WG), 0, st, L->descs, L->fin_items, ws, h);
    if ((rc = check_launch("kaon: k_fin launch"))) return rc;
  }
  hipLaunchKernelGGL(f1, dim3(L->n_row_items), dim3(KAON_WG), 0, st, L->descs, L->row_items, ws, h);
  if ((rc = check_launch("kaon: KProdigy pass-1 launch"))) return rc;
  if (h.flags & KAON_F_PD_BLOCKFAC) {
    // after k_pd1: the block-factored second moment reads its GC means
    PdBfacFn fb = pd_bfac_fn(h.p_dtype, h.g_dtype);
    if (!fb) return fail("kaon_kprodigy_pass1: unsupported dtype combination");
    hipLaunchKernelGGL(fb, dim3(L->n_tensors, 64), dim3(KAON_WG), 0, st, L->descs, ws, h);
    if ((rc = check_launch("kaon: KProdigy block-factored launch"))) return rc;
  }
  if ((h.flags & KAON_F_PD_STATS) && L->n_flat_items > 0) {
    hipLaunchKernelGGL(fs, dim3((L->n_flat_items + 3) / 4), dim3(KAON_WG), 0, st, L->descs, L->flat_items,
                       L->n_flat_items, ws, h);
    hipLaunchKernelGGL(k_pd_sfin, dim3((L->n_tensors + 3) / 4), dim3(KAON_WG), 0, st, L->descs, L->n_tensors, ws);
    if ((rc = check_launch("kaon: KProdigy statistics launch"))) return rc;
  }
  return 0;
}

int kaon_kprodigy_pass2(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  int rc = validate(L, hp, "kaon_kprodigy_pass2: null argument", true);
  if (rc) return rc;
  if (hp->flags & KAON_F_TORCH_ORDER)
    return fail("kaon_kprodigy_pass2: torch-order sums are built for the Adakaon (Nekaon, MSAM) and Lion steps");
  if (L->n_tensors <= 0 || L->n_elem_items <= 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  const bool mom = (h.flags & KAON_F_MOMENTUM) && h.codec != KAON_MOM_NONE;
  const int codec = mom ? h.codec : KAON_MOM_NONE;
  h.codec = codec;
  PdFn f5 = pd2_fn<5>(h.p_dtype, h.g_dtype, codec), f6 = pd2_fn<6>(h.p_dtype, h.g_dtype, codec);
  if (!f5 || !f6) return fail("kaon_kprodigy_pass2: unsupported dtype / codec combination");
  if (h.flags & KAON_F_CAUTIOUS) {
    hipLaunchKernelGGL(f5, dim3(L->n_elem_items), dim3(KAON_WG), 0, st, L->descs, L->elem_items, ws, h);
    if ((rc = check_launch("kaon: KProdigy keep-count launch"))) return rc;
  }
  hipLaunchKernelGGL(f6, dim3(L->n_elem_items), dim3(KAON_WG), 0, st, L->descs, L->elem_items, ws, h);
  return check_launch("kaon: KProdigy apply launch");
}

int kaon_lion_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream) {
  int rc = validate(L, hp, "kaon_lion_phases: null argument", true);
  if (rc) return rc;
  if (L->n_tensors <= 0 || L->n_row_items <= 0) return 0;
  if (hp->codec == KAON_MOM_NONE) return fail("kaon_lion_step: Lion always keeps a momentum buffer");
  hipStream_t st = (hipStream_t)stream;
  Ws ws{(float*)L->workspace};
  KaonHyper h = *hp;
  h.flags |= KAON_F_MOMENTUM;
  h.flags &= ~(KAON_F_NK_REMOVE | KAON_F_NK_CLIMB);
  const bool quant = h.codec == KAON_MOM_INT8 || h.codec == KAON_MOM_4BIT;
  if ((mask & (1u << 1)) && (h.flags & KAON_F_TORCH_ORDER)) {
    const int e = torch_phases(*L, ws, h, 1u << 1, 1, st);
    if (e) return fail("kaon: torch-order GC mean launch", (hipError_t)e);
  } else if (mask & (1u << 1)) {
    if ((rc = launch_stats(*L, ws, h, 1, st))) return rc;
  }
  if ((mask & (1u << 5)) && ((h.flags & KAON_F_CAUTIOUS) || quant)) {
    if ((rc = launch_elem<KAON_OPT_LION, 5>(*L, ws, h, h.codec, st))) return rc;
  }
  if (mask & (1u << 6)) {
    if ((rc = launch_elem<KAON_OPT_LION, 6>(*L, ws, h, h.codec, st))) return rc;
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
                     *hp, factor, bound, stream_id, (const float*)nullptr);
  return check_launch("kaon: msam launch");
}

int kaon_msam_apply_tensor(const KaonLaunch* L, const KaonHyper* hp, float signed_rho, float eps,
                           uint32_t stream_id, void* stream) {
  int rc = validate(L, hp, "kaon_msam_apply_tensor: null argument");
  if (rc) return rc;
  if (L->n_tensors <= 0) return 0;
  if (stream_id > 2) return fail("kaon_msam_apply_tensor: stream_id must be 0, 1 or 2");
  MsamFn fn = msam_fn(hp->p_dtype, hp->codec);
  if (!fn) return fail("kaon_msam_apply_tensor: needs a momentum codec");
  hipLaunchKernelGGL(fn, dim3(L->n_flat_items), dim3(KAON_WG), 0, (hipStream_t)stream, L->descs, L->flat_items,
                     *hp, signed_rho, eps, stream_id, (const float*)L->workspace);
  return check_launch("kaon: msam tensor-norm launch");
}

int kaon_gc_writeback(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  int rc = validate(L, hp, "kaon_gc_writeback: null argument", true);
  if (rc) return rc;
  if (L->n_tensors <= 0 || L->n_row_items <= 0 || !(hp->flags & KAON_F_GC)) return 0;
  if (hp->flags & KAON_F_SRC_O) return fail("kaon_gc_writeback: the row items read O, not the gradient");
  auto fn = hp->g_dtype == KAON_BF16 ? k_gc_write<KAON_BF16>
            : hp->g_dtype == KAON_F16 ? k_gc_write<KAON_F16> : k_gc_write<KAON_F32>;
  hipLaunchKernelGGL(fn, dim3(L->n_row_items * KAON_RUN), dim3(KAON_WG), 0, (hipStream_t)stream, L->descs,
                     L->row_items, Ws{(float*)L->workspace});
  return check_launch("kaon: gc writeback launch");
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

// The apply's HBM access mix without its arithmetic: per 8-element chunk, read
// 16 B of bf16 g, 16 B of bf16 p and 8 B of int8 m, write p and m back (5:3
// read:write, 8 B per element), non-temporal like the apply's streams.  p and m
// are changed by an integer add so no access can be dropped.
__global__ __launch_bounds__(KAON_WG) void k_apply_mix(const ku4* __restrict__ g_, ku4* __restrict__ p_,
                                                       ku2* __restrict__ m_, int64_t nch) {
  const KAON_G ku4* g = G(g_);
  KAON_G ku4* p = G(p_);
  KAON_G ku2* m = G(m_);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + stride < nch; i += 2 * stride) {
    const ku4 ga = ld_stream<true>(g + i), gb = ld_stream<true>(g + i + stride);
    ku4 pa = ld_stream<true>(p + i), pb = ld_stream<true>(p + i + stride);
    ku2 ma = ld_stream<true>(m + i), mb = ld_stream<true>(m + i + stride);
    pa.x += ga.x; pa.y += ga.y; pa.z += ga.z; pa.w += ga.w;
    pb.x += gb.x; pb.y += gb.y; pb.z += gb.z; pb.w += gb.w;
    ma.x += 1u; ma.y += 1u; mb.x += 1u; mb.y += 1u;
    st_stream(p + i, pa);
    st_stream(p + i + stride, pb);
    st_stream(m + i, ma);
    st_stream(m + i + stride, mb);
  }
  for (; i < nch; i += stride) {
    const ku4 ga = ld_stream<true>(g + i);
    ku4 pa = ld_stream<true>(p + i);
    ku2 ma = ld_stream<true>(m + i);
    pa.x += ga.x; pa.y += ga.y; pa.z += ga.z; pa.w += ga.w;
    ma.x += 1u; ma.y += 1u;
    st_stream(p + i, pa);
    st_stream(m + i, ma);
  }
}

int kaon_apply_ceiling(const void* g, void* p, void* m, int64_t n, void* stream) {
  if (n <= 0) return 0;
  if ((n & 7) || (((uintptr_t)g | (uintptr_t)p) & 15) || ((uintptr_t)m & 7))
    return fail("kaon_apply_ceiling: needs n % 8 == 0, 16-byte aligned g and p, 8-byte aligned m");
  const int64_t nch = n / 8;
  int64_t grid = (nch + KAON_WG * 2 - 1) / (KAON_WG * 2);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_apply_mix, dim3((unsigned)grid), dim3(KAON_WG), 0, (hipStream_t)stream, (const ku4*)g,
                     (ku4*)p, (ku2*)m, nch);
  return check_launch("kaon_apply_ceiling");
}

int kaon_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (bytes <= 0) return 0;
  if ((bytes & 15) || (((uintptr_t)src | (uintptr_t)dst) & 15)) return fail("kaon_copy: needs 16-byte alignment");
  const int64_t n16 = bytes / 16;
  // the fastest configuration of a size sweep on gfx950: 4 vectors per thread
  // per round, up to 65536 workgroups, non-temporal accesses
  int64_t g = (n16 + KAON_WG * 4 - 1) / (KAON_WG * 4);
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(k_copy, dim3((unsigned)g), dim3(KAON_WG), 0, (hipStream_t)stream, (const ku4*)src, (ku4*)dst,
                     n16);
  return check_launch("kaon_copy");
}

}  // extern "C"
