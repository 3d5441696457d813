// kaon_fast.hip -- the specialized phase-5/6 kernels (k_fast) of the fused
// optimizer step and their dispatch table.  A translation unit of its own so
// the library's kernels compile in parallel; kaon_step.hip launches them
// through fast_kernel().  Semantics per element: src/kaon/adakaon.py:968-1014,
// src/kaon/lion.py:454-485, src/kaon/msam.py:202-235 (Nekaon's fused removal
// and climb), src/kaon/adapnm.py:1209-1275, src/kaon/adamuon.py:557-593.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kaon_common.h"

using namespace kaon;

namespace {

// =============================================================== fast path
// Phases 5 and 6 specialized at compile time for bf16 params and grads,
// stochastic-rounding writes and 16-byte-aligned rows: every full 8-element
// chunk runs straight-line code; only a row's partial last chunk takes the
// generic per-element route.  FLAGS: bit 0 GC, 1 cautious, 2 weight decay,
// 3 Nekaon removal, 4 Nekaon climb.

// int8 requant code of mf with r = RN64(1/scale), as a float in [-127, 127]
__device__ __forceinline__ float q_int8(float mf, double r) {
  const float x = rintf(div_r64(mf, r));
  return fminf(fmaxf(x, -127.0f), 127.0f);
}

// Four int8 codes (floats in [-127, 127]) as the stored little-endian bytes:
// code + 128 is exact in [1, 255]; v_cvt_pk_u8_f32 inserts each byte and the
// xor turns offset-binary into two's complement.
__device__ __forceinline__ uint32_t pack_int8x4(float a, float b, float c, float d) {
  uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(a + 128.0f, 0, 0u);
  w = __builtin_amdgcn_cvt_pk_u8_f32(b + 128.0f, 1, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(c + 128.0f, 2, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(d + 128.0f, 3, w);
  return w ^ 0x80808080u;
}

// Per-tensor values of a fast slice, read from its descriptor once per
// workgroup.  Offsets inside the tensor are 32-bit (the planner keeps tensors
// of more than 2^31 elements off this kernel), so every access is a uniform
// base plus a 32-bit byte offset, and nothing is reloaded after a store.
struct FastCtx {
  const KAON_G uint8_t* g;       // bf16 grads
  KAON_G uint8_t* gw;            // the same, written by the apply under FF_GCW
  bool gcw;                      // ... for tensors whose gc_write is set
  KAON_G uint8_t* p;             // bf16 params
  KAON_G uint8_t* m;             // momentum codes or bf16 momentum
  KAON_G uint8_t* msc;           // momentum scales (per row or per block)
  const KAON_G uint8_t* cf;      // column factors (Adakaon)
  KAON_G uint8_t* bamax;         // 4-bit: per-block |m| maximum
  KAON_G uint8_t* boldsc;        // 4-bit: per-block scale before the step
  const KAON_G uint16_t* nz[3];  // injected noise streams, or null
  const KAON_G uint8_t* m2;      // AdaPNM: the negative buffer (read only)
  const KAON_G uint8_t* m2sc;    // AdaPNM: its scales
  const KAON_G uint8_t* o;       // AdaMuon: the orthogonal factor O (bf16, row-major like g)
  uint32_t tid;                  // Philox tensor id
  int bsh;                       // 4-bit: log2 of the block size
  int GL;                        // 4-bit: lanes per block
  bool xrow;                     // 4-bit: blocks cross rows (C % block != 0)
};

// noise8 of the chunk at element e0 < 2^31 (the counter's high word is 0).
__device__ __forceinline__ void noise8_u32(uint64_t seed, uint32_t step, uint32_t tid, uint32_t stream, uint32_t e0,
                                           const KAON_G uint16_t* inj, uint32_t w[8]) {
  if (inj) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w[i] = inj[e0 + i];
      settle(w[i]);
    }
    return;
  }
  uint32_t c[4] = {e0 >> 3, 0u, tid, stream};
  philox10(c, (uint32_t)seed, step);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[2 * i] = c[i] & 0xFFFFu;
    w[2 * i + 1] = c[i] >> 16;
  }
}

// noise8_u32 with each 16-bit value in the high half of its word (the random
// operand of v_cvt_sr_bf16_f32).  The instruction reads only bits 31:16 of
// that operand (a device check over every bf16 high half with random, all-ones
// and carry-boundary low halves found no difference from the masked word), so
// the odd element's word is the Philox word itself, its low half unmasked;
// sr_chunk's NaN path shifts the noise down and never sees the low half.
__device__ __forceinline__ void noise8_hi(uint64_t seed, uint32_t step, uint32_t tid, uint32_t stream, uint32_t e0,
                                          const KAON_G uint16_t* inj, uint32_t w[8]) {
  if (inj) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w[i] = (uint32_t)inj[e0 + i] << 16;
      settle(w[i]);
    }
    return;
  }
  uint32_t c[4] = {e0 >> 3, 0u, tid, stream};
  philox10(c, (uint32_t)seed, step);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[2 * i] = c[i] << 16;
    w[2 * i + 1] = c[i];
  }
}

typedef __bf16 kbf16x2 __attribute__((ext_vector_type(2)));

// The SR bit trick of eight values, as packed bf16 pairs.  v_cvt_sr_bf16_f32
// adds the high half of its random operand to the fp32 bits and truncates,
// which is the trick ((bits(x) + noise) with the low half cleared) for every
// x that is not NaN; it was compared with the trick on the device over every
// bf16 high half with noise around the carry boundary.  For a NaN the trick
// gives inf (a NaN whose payload sits in the low half plus a carry-free noise)
// or 0x7FC0, the instruction some NaN, so a chunk with a NaN anywhere in the
// wave takes the trick itself.  nzh: noise in the high halves.
// CLEAN: the caller has shown that no x is NaN (no ballots); nan_out receives
// the wave's NaN ballot otherwise.
template <bool CLEAN = false>
__device__ __forceinline__ ku4 sr_chunk(const float x[8], const uint32_t nzh[8], uint64_t* nan_out = nullptr) {
  uint64_t nan = 0;
  if (!CLEAN) {
    // one unordered compare per pair: true where either value is NaN
#pragma unroll
    for (int i = 0; i < 8; i += 2) nan |= __builtin_amdgcn_ballot_w64(__builtin_isunordered(x[i], x[i + 1]));
  }
  if (nan_out) *nan_out = nan;
  uint32_t w[4];
  if (nan == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kbf16x2 v = {};
      v = __builtin_amdgcn_cvt_sr_bf16_f32(v, x[2 * i], nzh[2 * i], false);
      v = __builtin_amdgcn_cvt_sr_bf16_f32(v, x[2 * i + 1], nzh[2 * i + 1], true);
      w[i] = __builtin_bit_cast(uint32_t, v);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = pack_hi16(sr_word(x[2 * i], nzh[2 * i] >> 16), sr_word(x[2 * i + 1], nzh[2 * i + 1] >> 16));
  }
  return ku4{w[0], w[1], w[2], w[3]};
}

// Global loads of one chunk, issued a chunk ahead of its arithmetic.
struct FastIn {
  ku4 g, p, m16;
  ku2 m8;
  uint32_t m4;
  kf4 c0, c1;
  float bo, ba;  // 4-bit: block scale before the step, block |m| maximum
  ku4 n16;       // AdaPNM: the negative buffer (bf16, int8, 4-bit) and its 4-bit block scale
  ku2 n8;
  uint32_t n4;
  float bn;
  ku4 o;         // AdaMuon: O
};

// AdaMuon's keep count reads no momentum (the update is O's; the momentum of
// the raw grad was stepped and its absmax taken by the momentum pass)
template <int OPT, int PHASE>
constexpr bool fast_reads_m() {
  return !(OPT == KAON_OPT_ADAMUON && PHASE == 5);
}

// Which passes of the specialized kernel read the weights: the apply, and for
// Adakaon's coupled form of weight decay also the keep count (AdaPNM decays p
// in the apply only).
template <int OPT, int PHASE, int FLAGS>
constexpr bool fast_needs_p() {
  return PHASE == 6 || ((FLAGS & FF_WD) && OPT != KAON_OPT_ADAPNM);
}

template <int OPT, int PHASE, int CODEC, int FLAGS>
__device__ __forceinline__ void fast_load(FastIn& in, const FastCtx& X, uint32_t e0, uint32_t j0) {
  constexpr bool NEEDP = fast_needs_p<OPT, PHASE, FLAGS>();
  constexpr bool PNM = OPT == KAON_OPT_ADAPNM, MUON = OPT == KAON_OPT_ADAMUON;
  constexpr bool RM = fast_reads_m<OPT, PHASE>();
  const ku4 z4 = ku4{0u, 0u, 0u, 0u};
  in.g = ld_stream<true>((const KAON_G ku4*)(X.g + 2u * e0));
  in.p = NEEDP ? ld_stream<true>((const KAON_G ku4*)(X.p + 2u * e0)) : z4;
  in.o = MUON ? *(const KAON_G ku4*)(X.o + 2u * e0) : z4;
  in.m8 = RM && CODEC == KAON_MOM_INT8 ? ld_stream<true>((const KAON_G ku2*)(X.m + e0)) : ku2{0u, 0u};
  in.m4 = RM && CODEC == KAON_MOM_4BIT ? ld_stream<true>((const KAON_G uint32_t*)(X.m + (e0 >> 1))) : 0u;
  in.m16 = RM && CODEC == KAON_MOM_BF16 ? ld_stream<true>((const KAON_G ku4*)(X.m + 2u * e0)) : z4;
  in.n8 = PNM && CODEC == KAON_MOM_INT8 ? ld_stream<true>((const KAON_G ku2*)(X.m2 + e0)) : ku2{0u, 0u};
  in.n4 = PNM && CODEC == KAON_MOM_4BIT ? ld_stream<true>((const KAON_G uint32_t*)(X.m2 + (e0 >> 1))) : 0u;
  in.n16 = PNM && CODEC == KAON_MOM_BF16 ? ld_stream<true>((const KAON_G ku4*)(X.m2 + 2u * e0)) : z4;
  if (OPT == KAON_OPT_ADAKAON || PNM || MUON) {
    in.c0 = *(const KAON_G kf4*)(X.cf + 4u * j0);
    in.c1 = *(const KAON_G kf4*)(X.cf + 4u * j0 + 16u);
  } else {
    in.c0 = in.c1 = kf4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  in.bo = in.ba = in.bn = 0.0f;
  if (CODEC == KAON_MOM_4BIT && RM) {
    const uint32_t blk4 = (e0 >> X.bsh) * 4u;
    in.bo = *(const KAON_G float*)((PHASE == 5 ? X.msc : X.boldsc) + blk4);
    if (PHASE == 6) in.ba = *(const KAON_G float*)(X.bamax + blk4);
    if (PNM) in.bn = *(const KAON_G float*)(X.m2sc + blk4);
  }
}

// Completes the loads of `in` on every path (see settle), so that the
// branches consuming them leave nothing pending for the next prefetch to wait on.
template <int OPT, int PHASE, int CODEC, int FLAGS>
__device__ __forceinline__ void fast_settle(const FastIn& in) {
  constexpr bool NEEDP = fast_needs_p<OPT, PHASE, FLAGS>();
  constexpr bool PNM = OPT == KAON_OPT_ADAPNM, MUON = OPT == KAON_OPT_ADAMUON;
  constexpr bool RM = fast_reads_m<OPT, PHASE>();
  settle(in.g.x); settle(in.g.y); settle(in.g.z); settle(in.g.w);
  if (MUON) {
    settle(in.o.x); settle(in.o.y); settle(in.o.z); settle(in.o.w);
  }
  if (NEEDP) {
    settle(in.p.x); settle(in.p.y); settle(in.p.z); settle(in.p.w);
  }
  if (RM && CODEC == KAON_MOM_INT8) {
    settle(in.m8.x); settle(in.m8.y);
  }
  if (RM && CODEC == KAON_MOM_4BIT) {
    settle(in.m4); settle(in.bo);
    if (PHASE == 6) settle(in.ba);
  }
  if (RM && CODEC == KAON_MOM_BF16) {
    settle(in.m16.x); settle(in.m16.y); settle(in.m16.z); settle(in.m16.w);
  }
  if (PNM) {
    if (CODEC == KAON_MOM_INT8) {
      settle(in.n8.x); settle(in.n8.y);
    }
    if (CODEC == KAON_MOM_4BIT) {
      settle(in.n4); settle(in.bn);
    }
    if (CODEC == KAON_MOM_BF16) {
      settle(in.n16.x); settle(in.n16.y); settle(in.n16.z); settle(in.n16.w);
    }
  }
  if (OPT == KAON_OPT_ADAKAON || PNM || MUON) {
    settle(in.c0.x); settle(in.c0.y); settle(in.c0.z); settle(in.c0.w);
    settle(in.c1.x); settle(in.c1.y); settle(in.c1.z); settle(in.c1.w);
  }
}

// FAC1: clip divisor 1 (skip the exact division).  DQX: a wave some of whose
// momentum scales are too large for the fma dequant form (int8 q*scale; AdaPNM:
// either buffer's) or, with int8 / 4-bit momentum outside AdaPNM and AdaMuon,
// whose new scales or Nekaon factor are not below 2^120 (the NaN-safe clamps).  WLO: the momentum lerp weight is below 0.5 (its branch of
// torch's lerp).
template <int OPT, int PHASE, int CODEC, int FLAGS, bool FAC1, bool DQX, bool WLO>
__device__ __forceinline__ void fast_chunk(const FastCtx& X, const FastIn& in, const KaonHyper& hp, uint32_t e0,
                                           float mu, float rf, float oldsc, float m128, float negsc, float m128n,
                                           float newsc, double rnew, double rfac, double rden, int lane,
                                           uint32_t& keep, float& amax, float bnew4) {
  constexpr bool GC = FLAGS & FF_GC, CAUT = FLAGS & FF_CAUT, WD = FLAGS & FF_WD;
  constexpr bool NKR = FLAGS & FF_NKR, NKC = FLAGS & FF_NKC;
  constexpr bool MOM = CODEC != KAON_MOM_NONE;
  constexpr bool PNM = OPT == KAON_OPT_ADAPNM, MUON = OPT == KAON_OPT_ADAMUON;
  constexpr bool NEEDP = fast_needs_p<OPT, PHASE, FLAGS>();
  const ku4 gv4 = in.g, pv4 = in.p, mb16 = in.m16;
  const ku2 mi8 = in.m8;
  const uint32_t m4 = in.m4;
  float f[8];
  if (OPT == KAON_OPT_ADAKAON || PNM || MUON) {
    f[0] = in.c0.x; f[1] = in.c0.y; f[2] = in.c0.z; f[3] = in.c0.w;
    f[4] = in.c1.x; f[5] = in.c1.y; f[6] = in.c1.z; f[7] = in.c1.w;
  }
  // !DQX (int8, 4-bit): every lane's momentum scales are below 2^120 (the
  // caller's wave-wide test, with the new scales and a finite Nekaon factor in
  // the apply, and positive Nekaon / MSAM bounds).  Then each dequantized
  // momentum and each perturbation before its clamp is a number that is not
  // NaN: the clamps need no NaN case and take one v_med3_f32 (the median of
  // x, -b, b is the clamp for b > 0, +inf included), the climb's input is NaN
  // only where the update's was, and a code dequantizes as
  // fma(code, s, -128 s) / fma(code, s, -8 s), exact since -128 s / -8 s and
  // the sum are then one rounding of (code - 128) s / (code - 8) s.
  constexpr bool SANE = !DQX && (CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT) && !PNM && !MUON;
  // 4-bit: one block per chunk; the apply's new scale max(|m| max, 1e-12) / 7
  // comes from the caller (bnew4)
  float b_old = 1.0f, b_new = 1.0f;
  double b_r = 1.0;
  uint32_t blk4 = 0;  // byte offset of the chunk's block in the per-block arrays
  if (CODEC == KAON_MOM_4BIT) {
    blk4 = (e0 >> X.bsh) * 4u;
    b_old = in.bo;
    if (PHASE == 6) {
      b_new = bnew4;
      // SANE: 1.4e-13 < b_new < 2^120
      b_r = SANE ? rcp64_nr(b_new) : rcp64(b_new);
    }
  }
  float g[8], p[8];
  unpack8(gv4, g);
  if (NEEDP) unpack8(pv4, p);
  if (GC) {
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      float a0 = g[i] - mu, a1 = g[i + 1] - mu;
      rbf2(a0, a1);
      g[i] = a0;
      g[i + 1] = a1;
    }
  }
  // LAZY: the keep count of a step that removes the previous climb and decays
  // the weights (phase 5 with NKR and WD) reads p after the removal's
  // stochastic rounding, which is one of two bf16 neighbours of p + e.  The
  // cautious test is evaluated for both; the removal's noise is drawn only for
  // chunks where some element's keep bit depends on which one it is.  Exact,
  // and rare.
  constexpr bool LAZY = PHASE == 5 && CAUT && NKR && NEEDP && !PNM && !MUON;
  uint32_t nz0[8], nz1[8], nz2[8];
  // phase 6 rounds through sr_chunk (noise in the high halves); phase 5 only
  // uses the removal's noise, through sr_bf16
  if (NKR && NEEDP && !LAZY) {
    if (PHASE == 6)
      noise8_hi(hp.seed, hp.step, X.tid, 0u, e0, X.nz[0], nz0);
    else
      noise8_u32(hp.seed, hp.step, X.tid, 0u, e0, X.nz[0], nz0);
  }
  if (PHASE == 6) noise8_hi(hp.seed, hp.step, X.tid, 1u, e0, X.nz[1], nz1);
  if (PHASE == 6 && NKC) noise8_hi(hp.seed, hp.step, X.tid, 2u, e0, X.nz[2], nz2);

  float mold[8];
  // 4-bit: the codes as floats, from the bytes of the even and the odd nibbles
  uint32_t nlo = m4 & 0x0F0F0F0Fu, nhi = (m4 >> 4) & 0x0F0F0F0Fu;
  if (CODEC == KAON_MOM_4BIT) {
    // opaque to the optimizer: otherwise it folds each byte's extraction back
    // into a bit-field extract of m4 and a conversion (two instructions per
    // code instead of one v_cvt_f32_ubyteN)
    asm volatile("" : "+v"(nlo));
    asm volatile("" : "+v"(nhi));
  }
  const float b8 = -8.0f * b_old;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (CODEC == KAON_MOM_4BIT) {
      const float cv = (float)((((i & 1) ? nhi : nlo) >> (8 * (i >> 1))) & 0xFFu);
      mold[i] = SANE ? __fmaf_rn(cv, b_old, b8) : (cv - 8.0f) * b_old;
    } else if (CODEC == KAON_MOM_INT8) {
      const uint32_t w = i < 4 ? mi8.x : mi8.y;
      if (DQX)
        mold[i] = (float)(int8_t)(uint8_t)((w >> (8 * (i & 3))) & 0xFFu) * oldsc;
      else
        mold[i] = __fmaf_rn((float)(((w ^ 0x80808080u) >> (8 * (i & 3))) & 0xFFu), oldsc, m128);
    } else if (CODEC == KAON_MOM_BF16) {
      const uint32_t mw[4] = {mb16.x, mb16.y, mb16.z, mb16.w};
      const uint32_t w = mw[i >> 1];
      mold[i] = (i & 1) ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
    } else {
      mold[i] = 0.0f;
    }
  }
  // AdaPNM: the negative buffer, dequantized as the positive one
  float mng[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    mng[i] = 0.0f;
    if (!PNM) continue;
    if (CODEC == KAON_MOM_INT8) {
      const uint32_t w = i < 4 ? in.n8.x : in.n8.y;
      if (DQX)
        mng[i] = (float)(int8_t)(uint8_t)((w >> (8 * (i & 3))) & 0xFFu) * negsc;
      else
        mng[i] = __fmaf_rn((float)(((w ^ 0x80808080u) >> (8 * (i & 3))) & 0xFFu), negsc, m128n);
    } else if (CODEC == KAON_MOM_4BIT) {
      mng[i] = ((float)((in.n4 >> (4 * i)) & 0xFu) - 8.0f) * in.bn;
    } else if (CODEC == KAON_MOM_BF16) {
      const uint32_t nw[4] = {in.n16.x, in.n16.y, in.n16.z, in.n16.w};
      const uint32_t w = nw[i >> 1];
      mng[i] = (i & 1) ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
    }
  }
  float d[8], mf[8], of[8], xr[8];
  uint32_t mbits[8];
  if (MUON) unpack8(in.o, of);
  if (NKR && NEEDP) {
    const float nf_old = msam_nanfill(hp.nk_bound_old);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = mold[i] * hp.nk_k;
      xr[i] = p[i] + (SANE ? __builtin_amdgcn_fmed3f(x, -hp.nk_bound_old, hp.nk_bound_old)
                           : msam_e(x, hp.nk_bound_old, nf_old));
    }
    if (PHASE == 6) {
      unpack8(sr_chunk(xr, nz0), p);
    } else if (!LAZY) {
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = bf2f(sr_bf16(xr[i], nz0[i]));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float pw = p[i];
    if (MUON) {
      // the update is O's (factored, clipped, lr = 0.2 lr); the momentum of the
      // raw grad is requantized in the apply
      const float u = (of[i] * rf) * f[i];
      d[i] = (FAC1 ? u : div_r64(u, rfac)) * hp.lr;
      mf[i] = PHASE == 6 ? klerp_b<WLO>(mold[i], g[i], hp.w1) : 0.0f;
    } else if (PNM) {
      // this step's positive buffer (decay beta1^2), the pos-neg mix, the
      // factored preconditioner with the bias correction, clip and lr
      const float mfv = __fmaf_rn(hp.a1, g[i], mold[i] * hp.b1);
      const float pn = __fmaf_rn(hp.pn_neg, mng[i], mfv * hp.pn_pos) * hp.pn_rnorm;
      const float u = pn * ((rf * f[i]) * hp.bc2);
      d[i] = (FAC1 ? u : div_r64(u, rfac)) * hp.lr;
      mf[i] = mfv;
      if (CODEC == KAON_MOM_BF16) mbits[i] = f2bf(mfv);
    } else if (OPT == KAON_OPT_ADAKAON) {
      const float u = (g[i] * rf) * f[i];
      const float ud = (FAC1 ? u : div_r64(u, rfac)) * hp.lr;
      if (CODEC == KAON_MOM_BF16) {
        const uint32_t mb = f2bf(klerp_b<WLO>(mold[i], rbf(ud), hp.w1));
        mbits[i] = mb;
        mf[i] = bf2f(mb);
        d[i] = mf[i];
      } else if (MOM) {
        mf[i] = klerp_b<WLO>(mold[i], ud, hp.w1);
        d[i] = mf[i];
      } else {
        mf[i] = 0.0f;
        d[i] = ud;
      }
    } else {
      d[i] = ksign(__fmaf_rn(hp.a1, g[i], mold[i] * hp.b1));
      mf[i] = __fmaf_rn(hp.a2, g[i], mold[i] * hp.b2);
      if (CODEC == KAON_MOM_BF16) mbits[i] = f2bf(mf[i]);
    }
    if (WD && !PNM && !LAZY) d[i] = __fmaf_rn(hp.wdl, pw, d[i]);
  }
  if (LAZY) {
    // For finite x = p + e the removal's rounding gives one of two bf16 bit
    // patterns: lo (x with its low half cleared) or lo + 0x10000 (one bf16 ulp
    // further from zero, inf past the largest finite value); for x = +-inf it
    // gives lo, and for NaN a NaN, whose keep bit is 0.  The keep bit d g > 0
    // is evaluated for both patterns.  Where they agree on every lane the
    // rounding cannot change it (a NaN x agrees only when both are 0) and lo's
    // d stands in; otherwise the wave draws the noise and rounds exactly.
    // The wave's keep bits are counted from the ballots (lane 0 carries them).
    uint64_t dis = 0;
    uint32_t cnt = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lb = __float_as_uint(xr[i]) & 0xFFFF0000u;
      const float dlo = __fmaf_rn(hp.wdl, __uint_as_float(lb), d[i]);
      const float dhi = __fmaf_rn(hp.wdl, __uint_as_float(lb + 0x10000u), d[i]);
      const uint64_t ml = __builtin_amdgcn_ballot_w64(dlo * g[i] > 0.0f);
      dis |= ml ^ __builtin_amdgcn_ballot_w64(dhi * g[i] > 0.0f);
      cnt += (uint32_t)__builtin_popcountll(ml);
    }
    if (dis != 0) {
      noise8_u32(hp.seed, hp.step, X.tid, 0u, e0, X.nz[0], nz0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float dx = __fmaf_rn(hp.wdl, bf2f(sr_bf16(xr[i], nz0[i])), d[i]);
        keep += dx * g[i] > 0.0f ? 1u : 0u;
      }
    } else {
      keep += lane == 0 ? cnt : 0u;
    }
  }
  if (PHASE == 5) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (CAUT && !LAZY) keep += d[i] * g[i] > 0.0f ? 1u : 0u;
      // AdaPNM's absmax of the new positive buffer comes from its clip-sum pass,
      // AdaMuon's from its momentum pass
      if ((CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT) && !PNM && !MUON) amax = fmaxf(amax, fabsf(mf[i]));
    }
    return;
  }
  // ---- phase 6: requant, cautious, SR write (+ Nekaon climb)
  float mdq[8];
  float codes[8];  // 4-bit: the centred code in [-7, 7], as a float
  float xq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (CODEC == KAON_MOM_INT8) {
      xq[i] = q_int8(mf[i], rnew);
      mdq[i] = xq[i] * newsc;
    } else if (CODEC == KAON_MOM_4BIT) {
      float x = rintf(div_r64(mf[i], b_r));
      x = fminf(fmaxf(x, -7.0f), 7.0f);
      codes[i] = x;
      mdq[i] = x * b_new;
    } else if (CODEC == KAON_MOM_BF16) {
      mdq[i] = mf[i];
    } else {
      mdq[i] = 0.0f;
    }
  }
  float xs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float dd = d[i];
    if (CAUT) dd = div_r64(d[i] * (d[i] * g[i] > 0.0f ? 1.0f : 0.0f), rden);
    if (OPT == KAON_OPT_LION) dd = dd * hp.lr;
    // AdaPNM's decoupled decay p * (1 - lr wd), rounded to the param dtype
    const float pd = PNM && WD ? rbf(p[i] * hp.wdl) : p[i];
    xs[i] = pd - dd;
  }
  uint64_t nan_u = 0;
  ku4 ov = sr_chunk(xs, nz1, &nan_u);
  if (NKC) {
    float y[8];
    unpack8(ov, y);
    const float nf_new = msam_nanfill(hp.nk_bound_new);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = mdq[i] * (-hp.nk_k);
      y[i] = y[i] + (SANE ? __builtin_amdgcn_fmed3f(x, -hp.nk_bound_new, hp.nk_bound_new)
                         : msam_e(x, hp.nk_bound_new, nf_new));
    }
    // the update's values were not NaN: neither are these (a finite step added)
    ov = (SANE && nan_u == 0) ? sr_chunk<true>(y, nz2) : sr_chunk(y, nz2);
  }
  st_stream((KAON_G ku4*)(X.p + 2u * e0), ov);
  // Nekaon / MSAM applies test the launch flag at run time (X.gcw) rather than
  // taking a template variant of their own
  if (PHASE == 6 && ((FLAGS & FF_GCW) || NKR || NKC) && GC && X.gcw) {
    // the centralized gradient, already rounded to bf16 (its low halves are zero)
    ku4 gv;
    gv.x = pack_hi16(__float_as_uint(g[0]), __float_as_uint(g[1]));
    gv.y = pack_hi16(__float_as_uint(g[2]), __float_as_uint(g[3]));
    gv.z = pack_hi16(__float_as_uint(g[4]), __float_as_uint(g[5]));
    gv.w = pack_hi16(__float_as_uint(g[6]), __float_as_uint(g[7]));
    st_stream((KAON_G ku4*)(X.gw + 2u * e0), gv);
  }
  if (CODEC == KAON_MOM_INT8) {
    ku2 mv;
    mv.x = pack_int8x4(xq[0], xq[1], xq[2], xq[3]);
    mv.y = pack_int8x4(xq[4], xq[5], xq[6], xq[7]);
    st_stream((KAON_G ku2*)(X.m + e0), mv);
  } else if (CODEC == KAON_MOM_4BIT) {
    // byte k = (c_2k + 8) + 16 (c_2k+1 + 8) = 16 c_2k+1 + (c_2k + 136), exact small
    // integers, packed by v_cvt_pk_u8_f32
    uint32_t v = __builtin_amdgcn_cvt_pk_u8_f32(__fmaf_rn(codes[1], 16.0f, codes[0] + 136.0f), 0, 0u);
    v = __builtin_amdgcn_cvt_pk_u8_f32(__fmaf_rn(codes[3], 16.0f, codes[2] + 136.0f), 1, v);
    v = __builtin_amdgcn_cvt_pk_u8_f32(__fmaf_rn(codes[5], 16.0f, codes[4] + 136.0f), 2, v);
    v = __builtin_amdgcn_cvt_pk_u8_f32(__fmaf_rn(codes[7], 16.0f, codes[6] + 136.0f), 3, v);
    *(KAON_G uint32_t*)(X.m + (e0 >> 1)) = v;
    if ((e0 & ((1u << X.bsh) - 1u)) == 0u) *(KAON_G float*)(X.msc + blk4) = b_new;  // the block's first chunk
  } else if (CODEC == KAON_MOM_BF16) {
    ku4 mv;
    mv.x = mbits[0] | (mbits[1] << 16);
    mv.y = mbits[2] | (mbits[3] << 16);
    mv.z = mbits[4] | (mbits[5] << 16);
    mv.w = mbits[6] | (mbits[7] << 16);
    st_stream((KAON_G ku4*)(X.m + 2u * e0), mv);
  }
}

// Fast slices (the planner's fast_eligible tensors): factored, bf16 params and
// grads, stochastic rounding, 16-byte aligned rows with C % 8 == 0 and, for
// 4-bit, blocks of 8*G elements with G | 64 (blocks that cross rows take one
// atomic maximum per chunk instead of the lane-group reduction).
template <int OPT, int PHASE, int CODEC, int FLAGS>
__global__ __launch_bounds__(KAON_WG) void k_fast(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, Ws ws, KaonHyper hp) {
  constexpr bool CAUT = FLAGS & FF_CAUT;
  constexpr bool QUANT = CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT;
  constexpr bool PNM = OPT == KAON_OPT_ADAPNM, MUON = OPT == KAON_OPT_ADAMUON;
  __shared__ uint32_t keep_s[4];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const uint32_t C = (uint32_t)T.C;
  const int64_t n = T.n;
  const uint32_t nfull = C >> 3;  // full chunks per row
  const WaveRows wr = wave_rows(it);
  FastCtx X;
  X.g = (const KAON_G uint8_t*)G(T.g);
  X.gw = (KAON_G uint8_t*)G(const_cast<void*>(T.g));
  // the launch stores centralized gradients and this tensor is one of them
  X.gcw = T.gc_write != 0 && (hp.flags & KAON_F_GC_WRITE) != 0;
  X.p = (KAON_G uint8_t*)G(T.p);
  // AdaPNM: m is this step's positive buffer (m on odd steps, m2 on even ones)
  const bool swap = PNM && (hp.step & 1u) == 0u;
  X.m = (KAON_G uint8_t*)G(swap ? T.m2 : T.m);
  X.msc = (KAON_G uint8_t*)G(swap ? T.m2_scale : T.m_scale);
  X.m2 = (const KAON_G uint8_t*)G(swap ? T.m : T.m2);
  X.m2sc = (const KAON_G uint8_t*)G(swap ? T.m_scale : T.m2_scale);
  X.o = MUON ? (const KAON_G uint8_t*)G(ws.mo(T)) : nullptr;
  X.cf = (const KAON_G uint8_t*)ws.cf(T);
  X.bamax = (KAON_G uint8_t*)ws.bamax(T);
  X.boldsc = CODEC == KAON_MOM_4BIT ? (KAON_G uint8_t*)ws.boldsc(T, nblocks4(T)) : X.bamax;
#pragma unroll
  for (int s = 0; s < 3; ++s) X.nz[s] = G(T.noise[s]);
  X.tid = (uint32_t)T.tensor_id;
  // 4-bit blocks are 8*GL elements with GL | 64, a power of two
  X.bsh = CODEC == KAON_MOM_4BIT ? __builtin_ctz((uint32_t)T.block4) : 3;
  X.GL = CODEC == KAON_MOM_4BIT ? (int)(T.block4 >> 3) : 1;
  X.xrow = CODEC == KAON_MOM_4BIT && (T.C % T.block4) != 0;

  // clip divisor of the tensor (phase 4)
  const float fac = OPT == KAON_OPT_ADAKAON || PNM || MUON ? ws.scal(T)[0] : 1.0f;
  const double rfac = rcp64(fac);
  double rden = 1.0;
  if (PHASE == 6 && CAUT) {
    const uint32_t cnt = ((const KAON_G uint32_t*)ws.scal(T))[1];
    rden = rcp64(fmaxf((float)cnt / (float)n, 1e-8f));
  }
  uint32_t keep = 0;
  // Adakaon / Nekaon momentum lerp weight 1 - beta1 (Lion has no lerp, AdaPNM an fma)
  const bool wlo = fabsf(hp.w1) < 0.5f;
  // per-row values of the wave's rows, one row per lane
  const int nrows = (int)(wr.re - wr.rb);
  const int64_t rl = lane_row(wr.rb, nrows, wr.lane);
  const float mu_l = (FLAGS & FF_GC) && nrows > 0 ? ws.mu(T)[rl] : 0.0f;
  const float rf_l = (OPT == KAON_OPT_ADAKAON || PNM || MUON) && nrows > 0 ? ws.rf(T)[rl] : 1.0f;
  const float sc_l = CODEC == KAON_MOM_INT8 && nrows > 0
                         ? (PHASE == 5 ? *(const KAON_G float*)(X.msc + 4u * (uint32_t)rl) : ws.roldsc(T)[rl])
                         : 1.0f;
  const float ng_l = PNM && CODEC == KAON_MOM_INT8 && nrows > 0 ? *(const KAON_G float*)(X.m2sc + 4u * (uint32_t)rl)
                                                                : 1.0f;
  const float am_l = CODEC == KAON_MOM_INT8 && PHASE == 6 && nrows > 0 ? __uint_as_float(ws.ramax(T)[rl]) : 0.0f;
  settle(mu_l);
  settle(rf_l);
  settle(sc_l);
  settle(ng_l);
  settle(am_l);
  // Each row is worked on by L = T.fast_lanes consecutive lanes (a power of
  // two), so a wave covers P = 64 / L rows at a time (a row set); chunk
  // round k of a row is chunks [L k, L k + L) with lane group member cl
  // taking chunk cl + L k.  The wave walks (row set, round) positions in
  // order, issuing the loads of the next position before the arithmetic of
  // the current one.  Lanes of rows past the slice, and of chunks past the
  // row end, load a valid chunk of their row again and skip the arithmetic.
  const int lsh = __builtin_ctz((uint32_t)T.fast_lanes);
  const uint32_t L = 1u << lsh;
  const int P = 64 >> lsh;
  const int rounds = (int)((nfull + L - 1) >> lsh);
  const int nsets = (nrows + P - 1) / P;
  const int total = nsets * rounds;
  const int grp = wr.lane >> lsh;             // the lane's row inside a row set
  const uint32_t cl = (uint32_t)wr.lane & (L - 1u);
  FastIn buf0, buf1;
  if (total > 0) {
    const uint32_t c = min(cl, nfull - 1u);
    const uint32_t re = (uint32_t)(wr.rb + min(grp, nrows - 1)) * C;
    fast_load<OPT, PHASE, CODEC, FLAGS>(buf0, X, re + 8u * c, 8u * c);
  }
  int s = 0, k = 0;
  int rj = 0;        // the lane's row (index into the wave's rows), clamped
  bool valid = false;
  uint32_t rowe = 0;
  float mu = 0.0f, rf = 1.0f, oldsc = 1.0f, newsc = 1.0f, m128 = 0.0f, amax = 0.0f, negsc = 1.0f, m128n = 0.0f;
  double rnew = 1.0;
  bool dqf = true;
  // Nekaon / MSAM factors the fast clamp form allows (see fast_chunk): a factor
  // below 2^120 and positive bounds
  const bool nk_ok = fabsf(hp.nk_k) < 0x1p120f && (!(FLAGS & FF_NKR) || hp.nk_bound_old > 0.0f) &&
                     (!(FLAGS & FF_NKC) || hp.nk_bound_new > 0.0f);
  // One position: arithmetic on `cur`, loads of the next position into `nxt`.
  // Called with the two buffers alternating, so no register copies wait on
  // the loads in flight.
  auto step = [&](int t, const FastIn& cur, FastIn& nxt) {
    if (k == 0) {
      const int ri = s * P + grp;
      valid = ri < nrows;
      rj = min(ri, nrows - 1);
      rowe = (uint32_t)(wr.rb + rj) * C;
      mu = (FLAGS & FF_GC) ? __shfl(mu_l, rj) : 0.0f;
      rf = OPT == KAON_OPT_ADAKAON || PNM || MUON ? __shfl(rf_l, rj) : 1.0f;
      if (CODEC == KAON_MOM_INT8) {
        oldsc = __shfl(sc_l, rj);
        if (PNM) negsc = __shfl(ng_l, rj);
        if (PHASE == 6) {
          newsc = fmaxf(__shfl(am_l, rj), 1e-12f) / 127.0f;
          rnew = rcp64(newsc);
          if (valid && cl == 0) *(KAON_G float*)(X.msc + 4u * (uint32_t)(wr.rb + rj)) = newsc;
        }
      }
      m128 = -128.0f * oldsc;
      m128n = -128.0f * negsc;
      // fma(ub, sc, -128 sc) is the exact product q*sc while 128*sc is finite
      dqf = CODEC != KAON_MOM_INT8 || (fabsf(oldsc) < 0x1p120f && (!PNM || fabsf(negsc) < 0x1p120f));
      amax = 0.0f;
    }
    int sn = s, kn = k + 1;
    if (kn == rounds) {
      kn = 0;
      ++sn;
    }
    {
      const bool last = t + 1 == total;
      const int rn = last ? rj : min((sn * P) + grp, nrows - 1);
      const uint32_t cn = min(cl + L * (uint32_t)(last ? k : kn), nfull - 1u);
      fast_load<OPT, PHASE, CODEC, FLAGS>(nxt, X, (uint32_t)(wr.rb + rn) * C + 8u * cn, 8u * cn);
    }
    fast_settle<OPT, PHASE, CODEC, FLAGS>(cur);
    const uint32_t c = cl + L * (uint32_t)k;
    const bool full = valid && c < nfull;
    float camax = 0.0f;
    // 4-bit apply: the block's new scale max(|m| max, 1e-12) / 7, rounded once
    // (div_r64 by RN64(1/7) is the IEEE quotient)
    const float bnew4 = CODEC == KAON_MOM_4BIT && PHASE == 6 ? div_r64(fmaxf(cur.ba, 1e-12f), 1.0 / 7.0) : 1.0f;
    if (QUANT && !PNM && !MUON) {
      // the wave's scales against 2^120 (see fast_chunk), one ballot per chunk
      const float s0 = CODEC == KAON_MOM_4BIT ? cur.bo : oldsc;
      const float s1 = PHASE != 6 ? 0.0f : CODEC == KAON_MOM_4BIT ? bnew4 : newsc;
      const bool ok = fabsf(s0) < 0x1p120f && fabsf(s1) < 0x1p120f;
      dqf = __builtin_amdgcn_ballot_w64(!ok) == 0 && nk_ok;
    }
    if (full) {
      const uint32_t e0 = rowe + 8u * c;
      if (wlo) {
        if (fac == 1.0f && dqf)
          fast_chunk<OPT, PHASE, CODEC, FLAGS, true, false, true>(
              X, cur, hp, e0, mu, rf, oldsc, m128, negsc, m128n, newsc, rnew, rfac, rden, wr.lane, keep, camax, bnew4);
        else if (dqf)
          fast_chunk<OPT, PHASE, CODEC, FLAGS, false, false, true>(
              X, cur, hp, e0, mu, rf, oldsc, m128, negsc, m128n, newsc, rnew, rfac, rden, wr.lane, keep, camax, bnew4);
        else
          fast_chunk<OPT, PHASE, CODEC, FLAGS, false, true, true>(
              X, cur, hp, e0, mu, rf, oldsc, m128, negsc, m128n, newsc, rnew, rfac, rden, wr.lane, keep, camax, bnew4);
      } else {
        if (fac == 1.0f && dqf)
          fast_chunk<OPT, PHASE, CODEC, FLAGS, true, false, false>(
              X, cur, hp, e0, mu, rf, oldsc, m128, negsc, m128n, newsc, rnew, rfac, rden, wr.lane, keep, camax, bnew4);
        else if (dqf)
          fast_chunk<OPT, PHASE, CODEC, FLAGS, false, false, false>(
              X, cur, hp, e0, mu, rf, oldsc, m128, negsc, m128n, newsc, rnew, rfac, rden, wr.lane, keep, camax, bnew4);
        else
          fast_chunk<OPT, PHASE, CODEC, FLAGS, false, true, false>(
              X, cur, hp, e0, mu, rf, oldsc, m128, negsc, m128n, newsc, rnew, rfac, rden, wr.lane, keep, camax, bnew4);
      }
    }
    if (PHASE == 5 && QUANT && !PNM && !MUON) {
      if (CODEC == KAON_MOM_INT8) {
        amax = fmaxf(amax, camax);
      } else if (X.xrow) {
        // 4-bit blocks across rows (a block is still whole chunks): one atomic
        // maximum per chunk into the block's |m| maximum (zeroed by phase 1).
        // The old block scale kept for the apply is the one `cur` already holds:
        // loading it again here would wait on the next position's loads too
        // (loads complete in order), which undoes the prefetch.
        if (full) {
          const uint32_t e0c = rowe + c * 8u;
          const uint32_t blk4 = (e0c >> X.bsh) * 4u;
          if (camax > 0.0f) atomicMax((uint32_t*)(X.bamax + blk4), __float_as_uint(camax));
          if ((e0c & ((1u << X.bsh) - 1u)) == 0u) *(KAON_G float*)(X.boldsc + blk4) = cur.bo;
        }
      } else {
        // 4-bit: a block is GL consecutive chunks, GL | L, so its lanes are
        // one aligned group of GL lanes
        float a = camax;
        for (int o = X.GL / 2; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
        if (full && (wr.lane & (X.GL - 1)) == 0) {
          const uint32_t blk4 = ((rowe + c * 8u) >> X.bsh) * 4u;
          *(KAON_G uint32_t*)(X.bamax + blk4) = __float_as_uint(a);
          *(KAON_G float*)(X.boldsc + blk4) = cur.bo;
        }
      }
    }
    if (PHASE == 5 && CODEC == KAON_MOM_INT8 && !PNM && !MUON && kn == 0) {
      // row maxima of the set: reduce over each row's L lanes
      float a = amax;
      for (int o = (int)L / 2; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
      if (valid && cl == 0) {
        ws.ramax(T)[wr.rb + rj] = __float_as_uint(a);
        ws.roldsc(T)[wr.rb + rj] = oldsc;
      }
    }
    s = sn;
    k = kn;
  };
  for (int t = 0; t < total; t += 2) {
    step(t, buf0, buf1);
    if (t + 1 < total) step(t + 1, buf1, buf0);
  }
  if (PHASE == 5 && CAUT) {
    const uint32_t wsum = wave_sum_u32(keep);
    if (wr.lane == 0) keep_s[wr.w] = wsum;
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t tot = keep_s[0] + keep_s[1] + keep_s[2] + keep_s[3];
      if (tot) atomicAdd(ws.keep_ctr(T), tot);
    }
  }
}

// specialized kernels available: (opt, codec, flags) with flags among the
// defaults of the reference optimizers (GC and cautious on, WD on or off;
// Nekaon: the climb, plus the removal after the first step, WD on or off;
// MSAM norm="global": the removal alone)
template <int OPT, int PHASE, int CODEC>
ElemFn fast_by_flags(int ff) {
  if constexpr (OPT == KAON_OPT_ADAMUON) {
    // int8 / 4-bit momenta (requantized in the apply); GC is off by default
    if constexpr (CODEC != KAON_MOM_INT8 && CODEC != KAON_MOM_4BIT) return nullptr;
    switch (ff) {
      case FF_CAUT: return k_fast<OPT, PHASE, CODEC, FF_CAUT>;
      case FF_CAUT | FF_WD: return k_fast<OPT, PHASE, CODEC, FF_CAUT | FF_WD>;
    }
  }
  switch (ff) {
    case FF_GC | FF_CAUT: return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT>;
    case FF_GC | FF_CAUT | FF_WD: return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_WD>;
  }
  if constexpr (PHASE == 6 && (OPT == KAON_OPT_ADAKAON || OPT == KAON_OPT_LION)) {
    // Lion, and Adakaon off its fused path, leave p.grad centralized (the
    // reference's native path)
    switch (ff) {
      case FF_GC | FF_CAUT | FF_GCW: return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_GCW>;
      case FF_GC | FF_CAUT | FF_WD | FF_GCW: return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_WD | FF_GCW>;
    }
  }
  if constexpr (OPT == KAON_OPT_ADAKAON && CODEC != KAON_MOM_NONE) {
    // the Nekaon / MSAM kernels store the centralized gradient under a run-time
    // test of the launch flag: one kernel with or without the write
    if (ff & (FF_NKR | FF_NKC)) ff &= ~FF_GCW;
    // phase 5 reads the weights (and so the removal) only under weight decay
    switch (ff) {
      case FF_GC | FF_CAUT | FF_WD | FF_NKR:
        return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_WD | FF_NKR>;
    }
    if constexpr (PHASE == 6) {
      switch (ff) {
        case FF_GC | FF_CAUT | FF_NKR: return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_NKR>;
      }
      if constexpr (CODEC == KAON_MOM_INT8 || CODEC == KAON_MOM_4BIT) {
        switch (ff) {
          case FF_GC | FF_CAUT | FF_NKC:
            return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_NKC>;
          case FF_GC | FF_CAUT | FF_NKC | FF_NKR:
            return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_NKC | FF_NKR>;
          case FF_GC | FF_CAUT | FF_WD | FF_NKC:
            return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_WD | FF_NKC>;
          case FF_GC | FF_CAUT | FF_WD | FF_NKC | FF_NKR:
            return k_fast<OPT, PHASE, CODEC, FF_GC | FF_CAUT | FF_WD | FF_NKC | FF_NKR>;
        }
      }
    }
  }
  return nullptr;
}

template <int OPT, int PHASE>
ElemFn fast_fn(int codec, int ff) {
  if (PHASE == 5) {
    // the climb and the gradient write-back are phase-6 writes; the removal matters to
    // phase 5 only where it reads the weights (weight decay): drop the flags phase 5
    // does not look at
    ff &= ~(FF_NKC | FF_GCW);
    if (!(ff & FF_WD)) ff &= ~FF_NKR;
  }
  switch (codec) {
    case KAON_MOM_NONE: return OPT == KAON_OPT_ADAKAON ? fast_by_flags<OPT, PHASE, KAON_MOM_NONE>(ff) : nullptr;
    case KAON_MOM_BF16: return fast_by_flags<OPT, PHASE, KAON_MOM_BF16>(ff);
    case KAON_MOM_INT8: return fast_by_flags<OPT, PHASE, KAON_MOM_INT8>(ff);
    case KAON_MOM_4BIT: return fast_by_flags<OPT, PHASE, KAON_MOM_4BIT>(ff);
  }
  return nullptr;
}

}  // namespace

namespace kaon {

ElemFn fast_kernel(int opt, int phase, int codec, int ff) {
  switch (opt) {
    case KAON_OPT_ADAKAON: return phase == 5 ? fast_fn<KAON_OPT_ADAKAON, 5>(codec, ff) : fast_fn<KAON_OPT_ADAKAON, 6>(codec, ff);
    case KAON_OPT_LION: return phase == 5 ? fast_fn<KAON_OPT_LION, 5>(codec, ff) : fast_fn<KAON_OPT_LION, 6>(codec, ff);
    case KAON_OPT_ADAMUON: return phase == 5 ? fast_fn<KAON_OPT_ADAMUON, 5>(codec, ff) : fast_fn<KAON_OPT_ADAMUON, 6>(codec, ff);
    case KAON_OPT_ADAPNM: return phase == 5 ? fast_fn<KAON_OPT_ADAPNM, 5>(codec, ff) : fast_fn<KAON_OPT_ADAPNM, 6>(codec, ff);
  }
  return nullptr;
}

}  // namespace kaon
