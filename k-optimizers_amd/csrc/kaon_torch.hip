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
// rows.  mode 1 (Lion): GC means only.  GC is a template parameter and eps1 is
// added as eps1 or 0 (x*x >= +0, so adding +0 changes nothing): a term has no
// branch, so a leaf's loads all issue before its adds.
template <int GT, bool GC>
__global__ __launch_bounds__(KAON_WG) void k_trow(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws, KaonHyper hp,
                                                  int mode) {
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  zero_accumulators(T, it, ws, hp.codec);
  const void* gsrc = T.g;
  if (!T.factored) {
    if (mode == 0) stats_1d<GT>(T, gsrc, hp, nullptr, nullptr);
    return;
  }
  if (mode == 1 && !GC) return;
  const float eadd = (hp.flags & KAON_F_EPS) ? hp.eps1 : 0.0f;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = (int)(threadIdx.x & 63), half = lane >> 5, pos = lane & 31;
  const int64_t C = T.C, end = (int64_t)it.row0 + it.nrows;
  for (int64_t rb = (int64_t)it.row0 + 2 * w; rb < end; rb += 8) {
    // a half without a row of its own repeats the last one and stores nothing
    const bool own = rb + half < end;
    const int64_t r = own ? rb + half : end - 1;
    const int64_t off = r * C;
    float mu = 0.0f;
    if (GC) {
      const float s = tinner32(C, pos, [&](int64_t j) { return ldx<GT>(gsrc, off + j); });
      mu = round_to<GT>(s / (float)C);
      if (own && pos == 0) ws.mu(T)[r] = mu;
    }
    if (mode == 1) continue;
    const float s2 = tinner32(C, pos, [&](int64_t j) {
      float x = ldx<GT>(gsrc, off + j);
      if (GC) x = round_to<GT>(x - mu);
      return x * x + eadd;
    });
    if (own && pos == 0) G(T.row)[r] = klerp(G(T.row)[r], s2 / (float)C, hp.w2);
  }
}

// =============================================================== phase 2
// Finalize items, four one-wave workgroups each.  kind 0: columns [row0,
// row0 + nrows): the column sum of G^2 (+eps1) over the rows (ko_torch_outer_sum:
// a cascade down the rows for the blocks of 32 columns -- blocks of 4 when C < 8
// -- and four row slots for the columns after them), then col = lerp(col, sum /
// R, 1-beta2) and cf = 1/sqrt(col).  A lane takes eight adjacent columns.  With
// aligned rows of C % 8 == 0 it runs their cascades side by side from one
// 16-byte load per row (fp32: two); otherwise, and for the columns after the
// 32-column blocks, one column after another.  (Two or four columns per lane
// for the tallest tensors, to even out the lanes' work, measured slower: the
// pass is bound by its load instructions, and narrower loads issue more.)
// kind 1 (workgroup 0): the row EMA's mean in torch's row order, rf =
// 1/sqrt(row / mean).
constexpr int kTfinSub = 4;
constexpr int kTfinWG = 64;
constexpr int kTfinCols = 8;  // columns per lane
static_assert(kTfinSub * kTfinWG * kTfinCols == KAON_COLITEM, "a finalize item's columns");

// tcascade of K accumulator positions side by side: position c sums term(i)[c]
// over i with exactly tcascade's additions.  `load(i, raw)` issues row i's
// loads, `term(i, raw, q)` forms its K terms.  A leaf's sum starts from 0 and
// depends on no other leaf, so with 16-term leaves the loads run two leaves
// ahead of the additions (three register sets, every load issued
// unconditionally from a row inside the range): a lane waits for memory about
// once per three leaves rather than once per leaf.
template <int K, class Raw, class L, class F>
__device__ void tcascade_k(int64_t size, L load, F term, float out[K]) {
  const int lp0 = ceil_log2_u64((uint64_t)size) / 4;
  const int lp = lp0 > 4 ? lp0 : 4;
  const int64_t step = (int64_t)1 << lp, mask = step - 1;
  float a0[K], a1[K], a2[K], a3[K];
#pragma unroll
  for (int c = 0; c < K; ++c) a0[c] = a1[c] = a2[c] = a3[c] = 0.0f;
  auto add_row = [&](int64_t i, const Raw& r) {
    float q[K];
    term(i, r, q);
#pragma unroll
    for (int c = 0; c < K; ++c) a0[c] = a0[c] + q[c];
  };
  // the leaf ending at row i is done: into level 1, and on up the levels
  auto close_leaf = [&](int64_t i) {
#pragma unroll
    for (int c = 0; c < K; ++c) {
      a1[c] = a1[c] + a0[c];
      a0[c] = 0.0f;
    }
    if ((i & (mask << lp)) == 0) {
#pragma unroll
      for (int c = 0; c < K; ++c) {
        a2[c] = a2[c] + a1[c];
        a1[c] = 0.0f;
      }
      if ((i & (mask << (2 * lp))) == 0) {
#pragma unroll
        for (int c = 0; c < K; ++c) {
          a3[c] = a3[c] + a2[c];
          a2[c] = 0.0f;
        }
      }
    }
  };
  int64_t i = 0;
  if (lp == 4) {
    const int64_t nleaf = size >> 4;
    if (nleaf > 0) {
      Raw r0[16], r1[16], r2[16];
      auto ld_leaf = [&](int64_t l, Raw(&r)[16]) {
        const int64_t b = (l < nleaf ? l : nleaf - 1) * 16;
#pragma unroll
        for (int j = 0; j < 16; ++j) load(b + j, r[j]);
      };
      auto do_leaf = [&](int64_t l, const Raw(&r)[16]) {
#pragma unroll
        for (int j = 0; j < 16; ++j) add_row(l * 16 + j, r[j]);
        close_leaf((l + 1) * 16);
      };
      ld_leaf(0, r0);
      ld_leaf(1, r1);
      for (int64_t l = 0; l < nleaf; l += 3) {
        ld_leaf(l + 2, r2);
        do_leaf(l, r0);
        if (l + 1 >= nleaf) break;
        ld_leaf(l + 3, r0);
        do_leaf(l + 1, r1);
        if (l + 2 >= nleaf) break;
        ld_leaf(l + 4, r1);
        do_leaf(l + 2, r2);
      }
      i = nleaf * 16;
    }
  } else {
    while (i + step <= size) {
      for (int64_t j = 0; j < step; ++j) {
        Raw r;
        load(i + j, r);
        add_row(i + j, r);
      }
      i += step;
      close_leaf(i);
    }
  }
  for (; i < size; ++i) {
    Raw r;
    load(i, r);
    add_row(i, r);
  }
#pragma unroll
  for (int c = 0; c < K; ++c) out[c] = ((a0[c] + a1[c]) + a2[c]) + a3[c];
}

// One row's K grad values at the lane's columns, as loaded (16-bit grads
// packed two to a word).
template <int GT, int K>
struct TfRaw {
  uint32_t w[GT == KAON_F32 ? K : K / 2];
};

// The column sums of columns j0 .. j0 + K - 1 (vector path: aligned rows of C %
// 8 == 0, all K inside the 32-column blocks), col / cf written.  FUSE: the term
// x*x + eps1 as one fused multiply-add, the same bits for 16-bit x when eps1 is
// 0 or at least 2^-100 (x*x is then exact, or below half an ulp of eps1).
template <int GT, bool GC, int K, bool FUSE>
__device__ __forceinline__ void tfin_cols(const KaonTensor& T, const Ws& ws, const KaonHyper& hp, int64_t j0) {
  const int64_t R = T.R, C = T.C;
  const void* gsrc = T.g;
  const float eadd = (hp.flags & KAON_F_EPS) ? hp.eps1 : 0.0f;
  const KAON_G float* mu = ws.mu(T);
  constexpr int NW = GT == KAON_F32 ? K : K / 2;  // 32-bit words per row
  float cs[K];
  tcascade_k<K, TfRaw<GT, K>>(
      R,
      [&](int64_t i, TfRaw<GT, K>& r) {
        const KAON_G uint8_t* p =
            (const KAON_G uint8_t*)G(gsrc) + (i * C + j0) * (GT == KAON_F32 ? 4 : 2);
        if (NW == 8) {
          const ku4 v0 = *(const KAON_G ku4*)p, v1 = *(const KAON_G ku4*)(p + 16);
          r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
          r.w[4 % NW] = v1.x; r.w[5 % NW] = v1.y; r.w[6 % NW] = v1.z; r.w[7 % NW] = v1.w;
        } else if (NW == 4) {
          const ku4 v = *(const KAON_G ku4*)p;
          r.w[0] = v.x; r.w[1 % NW] = v.y; r.w[2 % NW] = v.z; r.w[3 % NW] = v.w;
        } else if (NW == 2) {
          const ku2 v = *(const KAON_G ku2*)p;
          r.w[0] = v.x; r.w[1 % NW] = v.y;
        } else {
          r.w[0] = *(const KAON_G uint32_t*)p;
        }
      },
      [&](int64_t i, const TfRaw<GT, K>& r, float q[K]) {
        const float m = GC ? mu[i] : 0.0f;
#pragma unroll
        for (int c = 0; c < K; c += 2) {
          float x[2];
#pragma unroll
          for (int h = 0; h < 2; ++h)
            x[h] = GT == KAON_F32 ? __uint_as_float(r.w[(c + h) % NW])
                                  : lp2f<GT>(h ? (r.w[(c >> 1) % NW] >> 16) : (r.w[(c >> 1) % NW] & 0xFFFFu));
          if (GC) {
            x[0] = x[0] - m;
            x[1] = x[1] - m;
            // bf16: the packed conversion, RNE as round_to for every value but
            // NaN (whose term makes the column sum NaN either way)
            if (GT == KAON_BF16) {
              rbf2(x[0], x[1]);
            } else {
              x[0] = round_to<GT>(x[0]);
              x[1] = round_to<GT>(x[1]);
            }
          }
          q[c] = FUSE ? __fmaf_rn(x[0], x[0], eadd) : x[0] * x[0] + eadd;
          q[c + 1] = FUSE ? __fmaf_rn(x[1], x[1], eadd) : x[1] * x[1] + eadd;
        }
      },
      cs);
#pragma unroll
  for (int c = 0; c < K; ++c) {
    const int64_t j = j0 + c;
    const float nc = klerp(G(T.col)[j], cs[c] / (float)R, hp.w2);
    G(T.col)[j] = nc;
    ws.cf(T)[j] = 1.0f / sqrtf(nc);
  }
}

// Columns j0 .. min(j0 + K, end) - 1 one at a time (any row layout).
template <int GT, bool GC>
__device__ void tfin_scalar(const KaonTensor& T, const Ws& ws, const KaonHyper& hp, int64_t j0, int k, int64_t end) {
  const int64_t R = T.R, C = T.C;
  const void* gsrc = T.g;
  const float eadd = (hp.flags & KAON_F_EPS) ? hp.eps1 : 0.0f;
  const KAON_G float* mu = ws.mu(T);
  const int64_t jd = C >= 8 ? (C / 32) * 32 : (C / 4) * 4;
  for (int64_t j = j0; j < j0 + k && j < end; ++j) {
    auto q = [&](int64_t i) {
      float x = ldx<GT>(gsrc, i * C + j);
      if (GC) x = round_to<GT>(x - mu[i]);
      return x * x + eadd;
    };
    float cs;
    if (j < jd) {
      cs = tcascade(R, q);
    } else {
      const int64_t size = R / 4;
      float ps[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) ps[s] = tcascade(size, [&](int64_t i) { return q(4 * i + s); });
      for (int64_t i = 4 * size; i < R; ++i) ps[0] = ps[0] + q(i);
      cs = ((ps[0] + ps[1]) + ps[2]) + ps[3];
    }
    const float nc = klerp(G(T.col)[j], cs / (float)R, hp.w2);
    G(T.col)[j] = nc;
    ws.cf(T)[j] = 1.0f / sqrtf(nc);
  }
}

template <int GT, bool GC>
__global__ __launch_bounds__(kTfinWG) void k_tfin(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  const KaonItem it = items[blockIdx.x / kTfinSub];
  const int sb = (int)(blockIdx.x % kTfinSub);
  const KaonTensor& T = D[it.tensor];
  const int64_t R = T.R, C = T.C;
  const int lane = (int)threadIdx.x;
  if (it.kind == 0) {
    const int64_t end = (int64_t)it.row0 + it.nrows;
    const int64_t j0 = (int64_t)it.row0 + ((int64_t)sb * kTfinWG + lane) * kTfinCols;
    if (j0 >= end) return;
    const int64_t jd = C >= 8 ? (C / 32) * 32 : (C / 4) * 4;
    // aligned rows of C % 8 == 0: the lane's eight columns lie in one aligned
    // vector of every row, and all inside the 32-column blocks or all after them
    const float eadd = (hp.flags & KAON_F_EPS) ? hp.eps1 : 0.0f;
    if (T.vec_rows && C % 8 == 0 && j0 + kTfinCols <= jd) {
      if (GT != KAON_F32 && (eadd == 0.0f || eadd >= 0x1p-100f))
        tfin_cols<GT, GC, kTfinCols, GT != KAON_F32>(T, ws, hp, j0);
      else
        tfin_cols<GT, GC, kTfinCols, false>(T, ws, hp, j0);
    } else
      tfin_scalar<GT, GC>(T, ws, hp, j0, kTfinCols, end);
  } else {
    if (sb != 0) return;
    const KAON_G float* row = G((const float*)T.row);
    // every lane of the wave returns the whole sum
    const float rm = tinner32(R, lane & 31, [&](int64_t i) { return row[i]; }) / (float)R;
    KAON_G float* rf = ws.rf(T);
    for (int64_t i = lane; i < R; i += kTfinWG) rf[i] = 1.0f / sqrtf(row[i] / rm);
  }
}

// =============================================================== phases 3-4
// The clip divisor max(||U|| / sqrt(n) / clip, 1) of each tensor (one workgroup
// per tensor), ||U||^2 as torch's norm kernel forms it: lane k of 8 a sequential
// fma chain over elements k, k+8, ... of the first n - n % 8, the 8 lanes added
// in order, the tail fma'd after.  U = (G' r) c (factored) or g / sqrt(v) (1-D),
// G' the GC'd gradient.  Blocks of kTcS chunks of 8 elements: waves 1-7 compute
// U of block b + 1 into one LDS buffer (chunk s of the block -> column s, element
// k -> row k) while lanes 0-7 of wave 0 run the chains over block b in the other.
// A wave64 fma issues every ~4.7 cycles on its SIMD (two independent chains in
// one wave measure the same 4.7 cycles per fma), so the chain is bound by its
// SIMD's VALU issue, and any other wave's VALU work on that SIMD slows it.  So:
// one workgroup per CU (LDS above half the CU's), and the waves that share the
// chain wave's SIMD (HW_ID) produce nothing.  The producers issue each block's
// loads two blocks ahead (two register sets), so an HBM round trip under load
// overlaps two blocks of chain steps, and the chain lanes read LDS a round
// ahead of their fma.
// s_getreg operand of HW_ID's SIMD_ID field (hwreg 4, offset 4, 2 bits)
constexpr int kHwIdSimd = ((2 - 1) << 11) | (4 << 6) | 4;
constexpr int kTcWG = 512;                 // threads of the clip workgroup (8 waves)
constexpr int kTcS = 1296;                 // chunks (chain steps) per block
constexpr int kTcLd = kTcS + 4;            // LDS row stride: the 8 chain rows fall in distinct banks
constexpr int kTcLook = 2;                 // rounds of 16 chain steps the LDS reads run ahead
constexpr int kTcProdMin = 6 * 64;         // producer threads when the chain wave's SIMD holds two waves
constexpr int kTcSlots = (kTcS + kTcProdMin - 1) / kTcProdMin;

// U of element e (the tail and chunks across rows).
template <int GT, bool GC>
__device__ __forceinline__ float tclip_u(const KaonTensor& T, const Ws& ws, int64_t e) {
  const float x = ldx<GT>(T.g, e);
  if (!T.factored) return x * (1.0f / sqrtf(G(T.v)[e]));
  const uint32_t r = (uint32_t)e / (uint32_t)T.C, j = (uint32_t)e - r * (uint32_t)T.C;
  const float xg = GC ? round_to<GT>(x - ws.mu(T)[r]) : x;
  return (xg * ws.rf(T)[r]) * ws.cf(T)[j];
}

// Workgroup barrier that orders LDS only.  __syncthreads() also fences global
// memory, which waits for every load in flight -- the producers' loads issued
// blocks ahead included; the block handoff needs only the LDS writes done.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A producer slot's raw loads for one chunk: the grad chunk (16-bit grads kept
// packed, two to a word), the column factors (or v), the row's GC mean and factor.
template <int GT>
struct TcRaw {
  uint32_t x[GT == KAON_F32 ? 8 : 4];
  float f[8];
  float mu, rf;
};

template <int GT>
__device__ __forceinline__ void tc_ldg(const void* g, int64_t c, bool vec, TcRaw<GT>& w) {
  if (GT == KAON_F32) {
    float x[8];
    ld8<KAON_F32>(g, c * 8, 8, vec, x);
#pragma unroll
    for (int i = 0; i < 8; ++i) w.x[i] = __float_as_uint(x[i]);
  } else if (vec) {
    const ku4 v = *(const KAON_G ku4*)G((const uint16_t*)g + c * 8);
    w.x[0] = v.x; w.x[1] = v.y; w.x[2] = v.z; w.x[3] = v.w;
  } else {
    const KAON_G uint16_t* b = G((const uint16_t*)g + c * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) w.x[i] = (uint32_t)b[2 * i] | ((uint32_t)b[2 * i + 1] << 16);
  }
}
template <int GT>
__device__ __forceinline__ float tc_x(const TcRaw<GT>& w, int i) {
  if (GT == KAON_F32) return __uint_as_float(w.x[i]);
  const uint32_t h = (i & 1) ? (w.x[i >> 1] >> 16) : (w.x[i >> 1] & 0xFFFFu);
  return lp2f<GT>(h);
}

// KIND 0: 1-D (u = g / sqrt(v)); 1: factored rows of whole chunks (C % 8 == 0);
// 2: chunks across rows (element by element).
template <int GT, bool GC, int KIND>
__device__ __forceinline__ void tc_load(const KaonTensor& T, const Ws& ws, int64_t c, uint32_t cpr, bool vec,
                                        TcRaw<GT>& w) {
  if (KIND == 0) {
    tc_ldg<GT>(T.g, c, vec, w);
    ld8<KAON_F32>(T.v, c * 8, 8, vec, w.f);
  } else if (KIND == 1) {
    const uint32_t r = (uint32_t)c / cpr, j0 = ((uint32_t)c - r * cpr) * 8u;
    tc_ldg<GT>(T.g, c, vec, w);
    ld8<KAON_F32>((const float*)ws.cf(T), j0, 8, vec, w.f);
    w.mu = GC ? ws.mu(T)[r] : 0.0f;
    w.rf = ws.rf(T)[r];
  }
}
template <int GT, bool GC, int KIND>
__device__ __forceinline__ void tc_u(const KaonTensor& T, const Ws& ws, int64_t c, const TcRaw<GT>& w, float u[8]) {
  if (KIND == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = tc_x<GT>(w, i) * (1.0f / sqrtf(w.f[i]));
  } else if (KIND == 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = tc_x<GT>(w, i);
      const float xg = GC ? round_to<GT>(x - w.mu) : x;
      u[i] = (xg * w.rf) * w.f[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = tclip_u<GT, GC>(T, ws, c * 8 + i);
  }
}

// The chain lanes' pass over `cnt` steps of one LDS row.  A full block is
// straight-line code, 16 steps per round with the four 16-byte reads of the
// round kTcLook ahead issued before this round's fma, pinned by a scheduling
// barrier, and one LDS wait per round (the chain wave issues an instruction per
// ~4 cycles, so a wait per read costs a fifth of the rate)
// (in a loop the reads of the round ahead made the waits of the round at hand
// wait for them too); the last block of a tensor, shorter, reads as it goes.
__device__ __forceinline__ void tc_round(float& acc, const kf4 (&v)[4]) {
  // one asm statement over the round's sixteen operands, so the compiler's LDS
  // wait before it is a single s_waitcnt for all four reads; v_fmac_f32 is the
  // fused multiply-add __fmaf_rn compiles to (one rounding)
  asm volatile(
      "v_fmac_f32 %0, %1, %1\n\tv_fmac_f32 %0, %2, %2\n\tv_fmac_f32 %0, %3, %3\n\tv_fmac_f32 %0, %4, %4\n\t"
      "v_fmac_f32 %0, %5, %5\n\tv_fmac_f32 %0, %6, %6\n\tv_fmac_f32 %0, %7, %7\n\tv_fmac_f32 %0, %8, %8\n\t"
      "v_fmac_f32 %0, %9, %9\n\tv_fmac_f32 %0, %10, %10\n\tv_fmac_f32 %0, %11, %11\n\t"
      "v_fmac_f32 %0, %12, %12\n\tv_fmac_f32 %0, %13, %13\n\tv_fmac_f32 %0, %14, %14\n\t"
      "v_fmac_f32 %0, %15, %15\n\tv_fmac_f32 %0, %16, %16"
      : "+v"(acc)
      : "v"(v[0].x), "v"(v[0].y), "v"(v[0].z), "v"(v[0].w), "v"(v[1].x), "v"(v[1].y), "v"(v[1].z), "v"(v[1].w),
        "v"(v[2].x), "v"(v[2].y), "v"(v[2].z), "v"(v[2].w), "v"(v[3].x), "v"(v[3].y), "v"(v[3].z), "v"(v[3].w));
}
__device__ __forceinline__ float tc_chain(const float* row, int cnt, float acc) {
  const kf4* r4 = (const kf4*)row;
  if (cnt == kTcS) {
    constexpr int NR = kTcS / 16, LA = kTcLook;
    kf4 v[LA + 1][4];
#pragma unroll
    for (int t = 0; t < LA; ++t)
#pragma unroll
      for (int k = 0; k < 4; ++k) v[t][k] = r4[t * 4 + k];
#pragma unroll
    for (int t = 0; t < NR; ++t) {
      if (t + LA < NR) {
#pragma unroll
        for (int k = 0; k < 4; ++k) v[(t + LA) % (LA + 1)][k] = r4[(t + LA) * 4 + k];
      }
      // keep the reads above the round's fma (the scheduler would sink them to their use)
      __builtin_amdgcn_sched_barrier(0);
      tc_round(acc, v[t % (LA + 1)]);
    }
    return acc;
  }
  int s = 0;
  for (; s + 4 <= cnt; s += 4) {
    const kf4 x = r4[s / 4];
    acc = __fmaf_rn(x.x, x.x, acc);
    acc = __fmaf_rn(x.y, x.y, acc);
    acc = __fmaf_rn(x.z, x.z, acc);
    acc = __fmaf_rn(x.w, x.w, acc);
  }
  for (; s < cnt; ++s) acc = __fmaf_rn(row[s], row[s], acc);
  return acc;
}

template <int GT, bool GC, int KIND>
__device__ __forceinline__ void tclip_body(const KaonTensor& T, const Ws& ws, const KaonHyper& hp, float* lds,
                                           const int* simd, int mates) {
  const int64_t n = T.n;
  const int64_t body = n - n % 8, nchunks = body / 8;
  const int64_t nblk = (nchunks + kTcS - 1) / kTcS;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = (int)(threadIdx.x & 63);
  const bool vec = T.vec_rows != 0;
  const uint32_t cpr = (uint32_t)(T.C / 8);
  // producer rank: the waves other than the chain wave's SIMD mates, in wave order,
  // when those cover a block in kTcSlots rounds; otherwise waves 1-7
  static_assert((kTcWG / 64 - 1) * 64 * kTcSlots >= kTcS, "seven producer waves cover a block");
  const bool skip_mates = (kTcWG / 64 - 1 - mates) * 64 * kTcSlots >= kTcS;
  int prank = -1, nprod = 0;
  for (int w = 1; w < kTcWG / 64; ++w) {
    if (skip_mates && simd[w] == simd[0]) continue;
    if (w == wave) prank = nprod;
    ++nprod;
  }
  const int q0 = prank * 64 + lane;
  const int nq = nprod * 64;
  // two register sets: block b's loads go into set b & 1 (indices fixed at compile time)
  TcRaw<GT> raw0[kTcSlots], raw1[kTcSlots];

  auto load_block = [&](int64_t b, TcRaw<GT>(&raw)[kTcSlots]) {
#pragma unroll
    for (int k = 0; k < kTcSlots; ++k) {
      const int s = q0 + nq * k;
      const int64_t c = b * kTcS + s;
      if (prank >= 0 && s < kTcS && c < nchunks) tc_load<GT, GC, KIND>(T, ws, c, cpr, vec, raw[k]);
    }
  };
  auto store_block = [&](int64_t b, const TcRaw<GT>(&raw)[kTcSlots]) {
    const int buf = (int)(b & 1);
#pragma unroll
    for (int k = 0; k < kTcSlots; ++k) {
      const int s = q0 + nq * k;
      if (prank < 0 || s >= kTcS) continue;
      const int64_t c = b * kTcS + s;
      float u[8];
      if (c < nchunks) {
        tc_u<GT, GC, KIND>(T, ws, c, raw[k], u);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) lds[(buf * 8 + i) * kTcLd + s] = u[i];
    }
  };
  // The chain wave and the producers run loops of their own with the same
  // barriers (one after the prologue, one per block), so no register holds a
  // chain value on one path and a load in flight on the other.
  if (wave != 0) {
    // iteration b: store block b + 1 (its loads, issued at iteration b - 2, are
    // in set (b + 1) & 1), then issue block b + 3's into the same set
    if (nblk > 0) {
      load_block(0, raw0);
      if (nblk > 1) load_block(1, raw1);
      store_block(0, raw0);
      if (nblk > 2) load_block(2, raw0);
    }
    lds_barrier();
    for (int64_t b = 0; b < nblk; b += 2) {
      if (b + 1 < nblk) store_block(b + 1, raw1);
      if (b + 3 < nblk) load_block(b + 3, raw1);
      lds_barrier();
      if (b + 1 >= nblk) break;
      if (b + 2 < nblk) store_block(b + 2, raw0);
      if (b + 4 < nblk) load_block(b + 4, raw0);
      lds_barrier();
    }
    return;
  }
  float acc = 0.0f;  // lane k < 8: chain k
  lds_barrier();
  for (int64_t b = 0; b < nblk; ++b) {
    if (lane < 8) {
      const int cnt = (int)min<int64_t>(kTcS, nchunks - b * kTcS);
      acc = tc_chain(lds + ((int)(b & 1) * 8 + lane) * kTcLd, cnt, acc);
    }
    lds_barrier();
  }
  float ss = __shfl(acc, 0);
#pragma unroll
  for (int k = 1; k < 8; ++k) ss = ss + __shfl(acc, k);
  for (int64_t e = body; e < n; ++e) {
    const float u = tclip_u<GT, GC>(T, ws, e);
    ss = __fmaf_rn(u, u, ss);
  }
  // clip_threshold 0 leaves the update unclipped
  if (lane == 0) ws.scal(T)[0] = hp.clip > 0.0f ? fmaxf((sqrtf(ss) / T.sqrt_n) / hp.clip, 1.0f) : 1.0f;
}

template <int GT, bool GC>
__global__ __launch_bounds__(kTcWG) void k_tclip(const KaonTensor* __restrict__ D, int32_t t0, int32_t t1, Ws ws,
                                                 KaonHyper hp) {
  __shared__ __align__(16) float lds[2 * 8 * kTcLd];
  __shared__ int simd[kTcWG / 64];
  // ranks [t0, t1) of the tensors by decreasing size: the longest first, their
  // chains are the phase's critical path
  const int rank = t0 + (int)blockIdx.x;
  if (rank >= t1) return;
  const KaonTensor& T = D[D[rank].by_size];
  if (T.n == 0) return;
  // each wave's SIMD (HW_ID bits 5:4); the chain wave's SIMD mates stay idle
  // unless more than two of the eight waves share that SIMD
  if ((threadIdx.x & 63) == 0) simd[threadIdx.x >> 6] = (int)((__builtin_amdgcn_s_getreg(kHwIdSimd) >> 4) & 3u);
  __syncthreads();
  int mates = 0;
  for (int w = 1; w < kTcWG / 64; ++w) mates += simd[w] == simd[0];
  // the tensor's chunk kind, uniform over the workgroup (GC only touches 2-D tensors)
  if (!T.factored) tclip_body<GT, false, 0>(T, ws, hp, lds, simd, mates);
  else if (T.C % 8 == 0) tclip_body<GT, GC, 1>(T, ws, hp, lds, simd, mates);
  else tclip_body<GT, GC, 2>(T, ws, hp, lds, simd, mates);
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
using TclipFn = void (*)(const KaonTensor*, int32_t, int32_t, Ws, KaonHyper);


template <int GT>
int torch_phases_gt(const KaonLaunch& L, Ws ws, const KaonHyper& h, uint32_t mask, int mode, hipStream_t st) {
  const bool gc = (h.flags & KAON_F_GC) != 0;
  if (mask & (1u << 1)) {
    TrowFn f = gc ? k_trow<GT, true> : k_trow<GT, false>;
    hipLaunchKernelGGL(f, dim3(L.n_row_items), dim3(KAON_WG), 0, st, L.descs, L.row_items, ws, h, mode);
  }
  if (mode == 0 && (mask & (1u << 2)) && L.n_fin_items > 0) {
    TfinFn f = gc ? k_tfin<GT, true> : k_tfin<GT, false>;
    hipLaunchKernelGGL(f, dim3(L.n_fin_items * kTfinSub), dim3(kTfinWG), 0, st, L.descs, L.fin_items, ws, h);
  }
  if (mode == 0 && (mask & (1u << 3)) && L.n_tensors > 0) {
    TclipFn f = gc ? k_tclip<GT, true> : k_tclip<GT, false>;
    hipLaunchKernelGGL(f, dim3(L.n_tensors), dim3(kTcWG), 0, st, L.descs, 0, L.n_tensors, ws, h);
  }
  return (int)hipGetLastError();
}

template <int GT>
int torch_clip_gt(const KaonLaunch& L, Ws ws, const KaonHyper& h, int32_t t0, int32_t t1, hipStream_t st) {
  if (t1 <= t0) return 0;
  TclipFn f = (h.flags & KAON_F_GC) ? k_tclip<GT, true> : k_tclip<GT, false>;
  hipLaunchKernelGGL(f, dim3(t1 - t0), dim3(kTcWG), 0, st, L.descs, t0, t1, ws, h);
  return (int)hipGetLastError();
}

}  // namespace

// Phases 1-4 of an Adakaon step (mode 0) or phase 1 of a Lion step (mode 1) in
// torch's order, for the phase bits of `mask` (1, 2, 3; phase 3 also leaves the
// clip divisor, so bit 4 has nothing left to do).  Returns a HIP status.
int torch_phases(const KaonLaunch& L, Ws ws, const KaonHyper& h, uint32_t mask, int mode, hipStream_t st) {
  const int gt = h.g_dtype;
  return gt == KAON_BF16  ? torch_phases_gt<KAON_BF16>(L, ws, h, mask, mode, st)
         : gt == KAON_F16 ? torch_phases_gt<KAON_F16>(L, ws, h, mask, mode, st)
                          : torch_phases_gt<KAON_F32>(L, ws, h, mask, mode, st);
}

// Phase 3 of an Adakaon step in torch's order for the tensors of size ranks
// [t0, t1) (descs[k].by_size).  Returns a HIP status.
int torch_clip(const KaonLaunch& L, Ws ws, const KaonHyper& h, int32_t t0, int32_t t1, hipStream_t st) {
  const int gt = h.g_dtype;
  return gt == KAON_BF16  ? torch_clip_gt<KAON_BF16>(L, ws, h, t0, t1, st)
         : gt == KAON_F16 ? torch_clip_gt<KAON_F16>(L, ws, h, t0, t1, st)
                          : torch_clip_gt<KAON_F32>(L, ws, h, t0, t1, st);
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
