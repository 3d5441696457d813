// kaon_ns.hip -- AdaMuon's Newton-Schulz quintic iteration on gfx950 MFMA.
//
// zeropower_via_newtonschulz5 (src/kaon/adamuon.py:97-118), per matrix:
//   x = bf16(M) (transposed when R > C, so x is m x k with m <= k)
//   x = x / (||x|| + 1e-7)
//   repeat steps:  A = x x^T;  B = b*A + c*(A A);  x = a*x + B x
// with (a, b, c) = (3.4445, -4.7750, 2.0315) and every torch op on bf16
// tensors rounding its result to bf16 (products accumulate in fp32).
//
// Layout: each tensor's iterate lives zero-padded to m_pad x k_pad (multiples
// of KAON_NS_TILE) in its workspace block.  Zero rows and columns stay zero
// through all three products, so the GEMMs run on whole tiles with no edge
// masks and the padding never reaches the result.
//
// GEMMs: matrices of at least 512 rows take 256 x 256 output tiles (k_ns_gemm2,
// 4 wave64 of 128 x 128, two LDS stages of K = 64), the rest 128 x 128 tiles
// (k_ns_gemm, 4 wave64 of 64 x 64); both on v_mfma_f32_32x32x16_bf16 with the
// next K step's global loads in flight while the MFMAs run.  Work items list
// (tensor, tile row, tile column) for every tensor of the plan, so one launch
// per product and tile size covers the whole parameter list; the planner lays
// the big tiles out per XCD.  A = x x^T and A A are "NT" products (both
// operands row-major along K; A is symmetric, so big tiles cover row <= column
// and mirror); B x reads x along its rows with the LDS transpose read.  The
// last iteration's B x writes the orthogonal factor O over M.
#include "kaon_ns.h"

#include <string>
#include <type_traits>

#include "kaon_device.h"

using namespace kaon;

void kaon_set_error(const std::string& s);

namespace {

constexpr int TILE = KAON_NS_TILE;  // 128
constexpr int TK = 64;              // K per LDS stage
constexpr int LDK = TK + 8;         // LDS row stride (bf16), breaks bank aliasing

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct NsBufs {
  uint16_t* mo;  // M, then O: [R, C]
  uint16_t* x0;  // iterate ping
  uint16_t* x1;  // iterate pong
  uint16_t* a;   // A = x x^T  [m_pad, m_pad]
  uint16_t* b;   // B          [m_pad, m_pad]
};

__device__ __forceinline__ int64_t r4(int64_t x) { return (x + 3) & ~int64_t(3); }

// Word offsets as kaon_plan lays the block out (kaon_plan.cpp ns_words).
__device__ __forceinline__ NsBufs ns_bufs(float* base, const KaonTensor& T) {
  float* p = base + T.ws_aux;
  NsBufs nb;
  nb.mo = (uint16_t*)p;
  p += r4((T.R * T.C + 1) / 2);
  const int64_t xw = r4((int64_t)T.m_pad * T.k_pad / 2), aw = r4((int64_t)T.m_pad * T.m_pad / 2);
  nb.x0 = (uint16_t*)p;
  p += xw;
  nb.x1 = (uint16_t*)p;
  p += xw;
  nb.a = (uint16_t*)p;
  p += aw;
  nb.b = (uint16_t*)p;
  return nb;
}

__device__ __forceinline__ uint32_t half_of(const ku4 v, int e) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return (e & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// 8 bf16 into row r, columns c .. c + 7 of a row-major matrix, the ones inside
// rows x cols only.  ALN: the row stride is a multiple of 8.
__device__ __forceinline__ void ns_st8(uint16_t* p, int64_t ld, int r, int c, int rows, int cols, bool aln, ku4 v) {
  if (r >= rows) return;
  KAON_G uint16_t* q = G(p) + (int64_t)r * ld + c;
  if (aln && c + 8 <= cols) {
    *(KAON_G ku4*)q = v;
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (c + e < cols) q[e] = (uint16_t)half_of(v, e);
}

// The epilogue term on a packed pair of bf16-valued products x0, x1 and the
// packed A / x pair ew, with torch's roundings of each bf16 operation:
// MODE 1: bf16(bf16(b A) + bf16(c x)), MODE 2: bf16(bf16(a x) + x).  nan is
// set where a result is NaN (the packed conversion keeps NaN as NaN).
template <int MODE>
__device__ __forceinline__ uint32_t ns_comb2(float x0, float x1, uint32_t ew, float ca, float cb, float cc,
                                             bool& nan) {
  float t0 = __uint_as_float(ew << 16), t1 = __uint_as_float(ew & 0xFFFF0000u);
  float s0, s1;
  if (MODE == 1) {
    t0 *= cb;
    t1 *= cb;
    rbf2(t0, t1);
    float u0 = cc * x0, u1 = cc * x1;
    rbf2(u0, u1);
    s0 = t0 + u0;
    s1 = t1 + u1;
  } else {
    t0 *= ca;
    t1 *= ca;
    rbf2(t0, t1);
    s0 = t0 + x0;
    s1 = t1 + x1;
  }
  nan |= __builtin_isunordered(s0, s1);
  return f2bf2(s0, s1);
}

template <int MODE>
__device__ __forceinline__ ku4 ns_comb8(ku4 xv, ku4 ev, float ca, float cb, float cc, bool& nan) {
  auto one = [&](uint32_t xw, uint32_t ew) {
    return ns_comb2<MODE>(__uint_as_float(xw << 16), __uint_as_float(xw & 0xFFFF0000u), ew, ca, cb, cc, nan);
  };
  return ku4{one(xv.x, ev.x), one(xv.y, ev.y), one(xv.z, ev.z), one(xv.w, ev.w)};
}

// A packed bf16 pair with every NaN made torch's 0x7FC0: the packed conversion
// leaves NaN payloads unspecified, and O is the factor the step goes on with.
__device__ __forceinline__ uint32_t ns_canon2(uint32_t w) {
  const uint32_t lo = (w & 0x7FFFu) > 0x7F80u ? 0x7FC0u : (w & 0xFFFFu);
  const uint32_t hi = ((w >> 16) & 0x7FFFu) > 0x7F80u ? 0x7FC0u : (w >> 16);
  return lo | (hi << 16);
}

// MODE 0: A = x x^T.  MODE 1: B = b*A + c*(A A).  MODE 2: x' = a*x + B x.
// FIN (MODE 2, the last iteration): x' goes straight to O [R, C] over M,
// transposed back when R > C, and the padding is dropped.
template <int MODE, bool FIN = false>
__global__ __launch_bounds__(256) void k_ns_gemm(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, float* ws, int parity,
                                                 float ca, float cb, float cc) {
  __shared__ __attribute__((aligned(16))) uint16_t As[TILE * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[TILE * LDK];
  const KaonItem it = items[blockIdx.x];
  const KaonTensor& T = D[it.tensor];
  const NsBufs nb = ns_bufs(ws, T);
  const int mp = T.m_pad, kp = T.k_pad;
  const uint16_t* xc = parity ? nb.x1 : nb.x0;
  uint16_t* xn = parity ? nb.x0 : nb.x1;
  const uint16_t* Aop = MODE == 0 ? xc : MODE == 1 ? nb.a : nb.b;
  const uint16_t* Bop = MODE == 1 ? nb.a : xc;
  const int lda = MODE == 0 ? kp : mp;
  const int ldb = MODE == 1 ? mp : kp;
  const int K = MODE == 0 ? kp : mp;
  uint16_t* out = MODE == 0 ? nb.a : MODE == 1 ? nb.b : xn;
  const int ldc = MODE == 2 ? kp : mp;
  const int row0 = it.row0 * TILE, col0 = it.nrows * TILE;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // staging registers: 4 x 16 B of each operand per thread per K step
  ku4 ra[4], rb[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int q = tid + 256 * s, r = q >> 3, kc = q & 7;
      ra[s] = *(const KAON_G ku4*)G(Aop + (int64_t)(row0 + r) * lda + k0 + kc * 8);
    }
    if (MODE != 2) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int q = tid + 256 * s, r = q >> 3, kc = q & 7;
        rb[s] = *(const KAON_G ku4*)G(Bop + (int64_t)(col0 + r) * ldb + k0 + kc * 8);
      }
    } else {
      // x tile: K rows (k0..k0+63) x 128 columns; a thread takes two adjacent
      // rows of 8 columns so its LDS writes pack row pairs into 32-bit words
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int q = tid + 256 * s, jc = q >> 5, tp = q & 31;
        const uint16_t* src = Bop + (int64_t)(k0 + 2 * tp) * ldb + col0 + jc * 8;
        rb[2 * s] = *(const KAON_G ku4*)G(src);
        rb[2 * s + 1] = *(const KAON_G ku4*)G(src + ldb);
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int q = tid + 256 * s, r = q >> 3, kc = q & 7;
      *(ku4*)&As[r * LDK + kc * 8] = ra[s];
    }
    if (MODE != 2) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int q = tid + 256 * s, r = q >> 3, kc = q & 7;
        *(ku4*)&Bs[r * LDK + kc * 8] = rb[s];
      }
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int q = tid + 256 * s, jc = q >> 5, tp = q & 31;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *(uint32_t*)&Bs[(jc * 8 + e) * LDK + 2 * tp] = half_of(rb[2 * s], e) | (half_of(rb[2 * s + 1], e) << 16);
      }
    }
  };

  gload(0);
  for (int k0 = 0; k0 < K; k0 += TK) {
    __syncthreads();  // the previous step's MFMAs are done with the LDS tiles
    lstore();
    __syncthreads();
    if (k0 + TK < K) gload(k0 + TK);
#pragma unroll
    for (int kk = 0; kk < TK; kk += 16) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *(const bf16x8*)&As[(wm * 64 + i * 32 + (lane & 31)) * LDK + kk + (lane >> 5) * 8];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bfr[j] = *(const bf16x8*)&Bs[(wn * 64 + j * 32 + (lane & 31)) * LDK + kk + (lane >> 5) * 8];
      // the transposed product of each 32 x 32 block (see the epilogue)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue: acc[i][j] holds block (i, j) transposed, so lane l has row l % 32
  // of the block, columns 8 (r / 4) + 4 (l / 32) + r % 4: 8-byte accesses
  const uint16_t* eop = MODE == 1 ? nb.a : xc;
  const int lde = MODE == 1 ? mp : kp;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = row0 + wm * 64 + i * 32 + (lane & 31);
        const int col = col0 + wn * 64 + j * 32 + 8 * g + 4 * (lane >> 5);
        uint64_t ev = 0;
        if (MODE != 0) ev = *(const KAON_G uint64_t*)G(eop + (int64_t)row * lde + col);
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float x0 = acc[i][j][4 * g + 2 * h], x1 = acc[i][j][4 * g + 2 * h + 1];
          if (MODE == 0) {
            w[h] = f2bf2(x0, x1);
          } else {
            rbf2(x0, x1);
            bool nan = false;  // the final store below makes every NaN 0x7FC0 itself
            w[h] = ns_comb2<MODE>(x0, x1, (uint32_t)(ev >> (32 * h)), ca, cb, cc, nan);
          }
          if (FIN) w[h] = ns_canon2(w[h]);
        }
        if (FIN) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int orow = T.ns_tr ? col + e : row, ocol = T.ns_tr ? row : col + e;
            if (orow < T.R && ocol < T.C) G(nb.mo)[(int64_t)orow * T.C + ocol] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
          }
        } else {
          *(KAON_G uint64_t*)G(out + (int64_t)row * ldc + col) = (uint64_t)w[0] | ((uint64_t)w[1] << 32);
        }
      }
}

// Big tiles: one 256 x 256 output tile per workgroup, 4 wave64 of 128 x 128
// (4 x 4 v_mfma_f32_32x32x16_bf16 tiles accumulating in AGPRs), K in steps of
// 64 through two LDS stages: the next step's global loads and LDS stores
// overlap the current step's MFMAs, one barrier per step.  Per step a wave
// reads 32 KiB of fragments for 64 MFMAs, so LDS stays below its bandwidth at
// full MFMA rate (a 64 x 64 wave tile needs more than LDS provides).  The
// symmetric products (MODE 0, 1) run on tiles with row <= column and also store
// the transposed tile: its elements are the same products summed in the same
// order, so the mirror is exact.  The epilogue goes through LDS so that every
// global access is 16 bytes.
constexpr int BT = 2 * TILE;     // 256
constexpr int BK = 64;           // K per stage
constexpr int BLD = BK + 8;      // LDS row stride (bf16): 144 B, 16-B aligned rows, no bank aliasing
constexpr int WLD = 128 + 8;     // epilogue staging row stride (bf16): a wave's 128 x 128 tile
// MODE 2 keeps x as it lies in memory, BK rows of K by BT columns, and reads its
// MFMA fragments with the LDS transpose read (ds_read_b64_tr_b16).  A 16-lane
// group reads 32 bytes from each of 4 consecutive rows, and the group 16
// columns on is served in the same LDS cycle: a row stride of 576 B (64 B past
// a multiple of 256) puts the two groups' 8 pieces in distinct banks.
constexpr int XLD = BT + 32;
static_assert(BK * XLD <= BT * BLD, "the x tile fits the B stage");
constexpr int NS_LDS = (2 * 2 * BT * BLD > 4 * 128 * WLD) ? 2 * 2 * BT * BLD : 4 * 128 * WLD;

template <int MODE, bool FIN = false>
__global__ __launch_bounds__(256) void k_ns_gemm2(const KaonTensor* __restrict__ D,
                                                  const KaonItem* __restrict__ items, float* ws, int parity,
                                                  float ca, float cb, float cc) {
  // K loop: [stage][A, B][BT][BLD]; epilogue: [wave][128][WLD]
  __shared__ __attribute__((aligned(16))) uint16_t lds[NS_LDS];
  const KaonItem it = items[blockIdx.x];
  if (it.tensor < 0) return;  // an idle item of a shorter XCD list
  const KaonTensor& T = D[it.tensor];
  const NsBufs nb = ns_bufs(ws, T);
  const int mp = T.m_pad, kp = T.k_pad;
  const uint16_t* xc = parity ? nb.x1 : nb.x0;
  uint16_t* xn = parity ? nb.x0 : nb.x1;
  const uint16_t* Aop = MODE == 0 ? xc : MODE == 1 ? nb.a : nb.b;
  const uint16_t* Bop = MODE == 1 ? nb.a : xc;
  const int lda = MODE == 0 ? kp : mp;
  const int ldb = MODE == 1 ? mp : kp;
  const int K = MODE == 0 ? kp : mp;
  uint16_t* out = MODE == 0 ? nb.a : MODE == 1 ? nb.b : xn;
  const int ldc = MODE == 2 ? kp : mp;
  const int row0 = it.row0 * BT, col0 = it.nrows * BT;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1;
  auto As = [&](int st) { return lds + (st * 2 + 0) * BT * BLD; };
  auto Bs = [&](int st) { return lds + (st * 2 + 1) * BT * BLD; };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // staging: 8 x 16 B of each operand per thread per step (256 rows x 64 K)
  constexpr int KC = BK / 8;     // 16-byte chunks per row per step
  constexpr int NS = BT * KC / 256;
  ku4 ra[NS], rb[NS];
  // DG: a diagonal tile of a symmetric product, whose two operands are the same
  // row panel -- it is loaded and stored once and both fragments read it
  auto gload = [&](int k0, auto dg) {
    constexpr bool DG = decltype(dg)::value;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int q = tid + 256 * s, r = q / KC, kc = q % KC;
      ra[s] = *(const KAON_G ku4*)G(Aop + (int64_t)(row0 + r) * lda + k0 + kc * 8);
    }
    if (MODE != 2) {
      if (DG) return;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int q = tid + 256 * s, r = q / KC, kc = q % KC;
        rb[s] = *(const KAON_G ku4*)G(Bop + (int64_t)(col0 + r) * ldb + k0 + kc * 8);
      }
    } else {
      // x: BK K rows x 256 columns, 16-byte chunks along its rows
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int q = tid + 256 * s, kr = q / (BT / 8), nc = q % (BT / 8);
        rb[s] = *(const KAON_G ku4*)G(Bop + (int64_t)(k0 + kr) * ldb + col0 + nc * 8);
      }
    }
  };
  auto lstore = [&](int st, auto dg) {
    constexpr bool DG = decltype(dg)::value;
    uint16_t* as = As(st);
    uint16_t* bs = Bs(st);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int q = tid + 256 * s, r = q / KC, kc = q % KC;
      *(ku4*)&as[r * BLD + kc * 8] = ra[s];
    }
    if (MODE != 2) {
      if (DG) return;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int q = tid + 256 * s, r = q / KC, kc = q % KC;
        *(ku4*)&bs[r * BLD + kc * 8] = rb[s];
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int q = tid + 256 * s, kr = q / (BT / 8), nc = q % (BT / 8);
        *(ku4*)&bs[kr * XLD + nc * 8] = rb[s];
      }
    }
  };

  // Fragments are double-buffered across the four 16-K sub-steps of a stage:
  // sub-step t's MFMAs run while t + 1's fragments load, and the scheduling
  // groups below pin that interleave (left alone, the compiler loads each
  // fragment right before its MFMAs and one wave per SIMD exposes every LDS
  // latency).  The next stage's global loads are spread over sub-step 0 and
  // its LDS stores over sub-step 3; the last step re-loads its own K range so
  // that the step stays one basic block.
  bf16x8 fa[2][4], fb[2][4];
  auto lfrag = [&](int buf, const uint16_t* as, const uint16_t* bs, int kk) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[buf][i] = *(const bf16x8*)&as[(wm * 128 + i * 32 + (lane & 31)) * BLD + kk + (lane >> 5) * 8];
    if (MODE != 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[buf][j] = *(const bf16x8*)&bs[(wn * 128 + j * 32 + (lane & 31)) * BLD + kk + (lane >> 5) * 8];
    } else {
      // Lane l needs x[kk + 8 (l / 32) + 0..7][n0 + l % 32].  In each group of 16
      // lanes the transpose read gives lane i element i % 4 of the 8-byte chunks
      // of lanes i / 4 + 4 t (t = 0..3); lane s of the group points at row
      // kbase + s / 4, columns nbase + 4 (s % 4) .. + 3, so lane i receives
      // x[kbase + t][nbase + i]: four K values of its column per read, two reads.
      const int g = lane >> 4, sl = lane & 15;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nbase = wn * 128 + j * 32 + 16 * (g & 1), kbase = kk + 8 * (g >> 1);
        const uint16_t* p = bs + (kbase + (sl >> 2)) * XLD + nbase + 4 * (sl & 3);
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p + 4 * XLD));
        const v8s c = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        fb[buf][j] = __builtin_bit_cast(bf16x8, c);
      }
    }
  };
  // the transposed product of each 32 x 32 block, so that a lane ends up with
  // 4-column runs of one output row (see the epilogue)
  auto mma = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[buf][j], fa[buf][i], acc[i][j], 0, 0, 0);
  };
  constexpr int SG_MFMA = 0x008, SG_VMEM_RD = 0x020, SG_DS_RD = 0x100, SG_DS_WR = 0x200;
  constexpr int NWR = 2 * NS;  // LDS store instructions per step
  constexpr int RD2 = MODE == 2 ? 2 : 1;  // MODE 2: 12 fragment reads per sub-step, else 8

  // B x's epilogue adds a x at the output position: rows [wr0, wr0 + 128) of x,
  // the K rows this wave's tile streams at K offsets wr0 and wr0 + 64.  The
  // first 64 of them (ev[0..15]) are copied out of the LDS stage at K offset
  // wr0; the rest are read from memory after the loop (keeping all 128 rows
  // would take 128 more VGPRs than the wave has).
  const int wr0 = row0 + wm * 128, wc0 = col0 + wn * 128;
  ku4 ev[32];
  auto kloop = [&](auto dg) {
    constexpr bool DG = decltype(dg)::value;
    constexpr int VMS = DG ? NS / 8 : 2 * NS / 8;  // global loads per scheduling slot of sub-step 0
    constexpr int WRS = DG ? NWR / 16 : NWR / 8;   // LDS stores per slot of sub-step 3
    const int nk = K / BK;
    gload(0, dg);
    lstore(0, dg);
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
      const int cur = ks & 1;
      const uint16_t* as = As(cur);
      const uint16_t* bs = DG ? As(cur) : Bs(cur);
      if (MODE == 2 && ks * BK == wr0) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int i = u >> 3, j = (u >> 1) & 3, q = lane + 64 * (u & 1);
          ev[u] = *(const ku4*)&bs[(i * 32 + (q >> 2)) * XLD + wn * 128 + j * 32 + (q & 3) * 8];
        }
      }
      lfrag(0, as, bs, 0);
      gload(min(ks + 1, nk - 1) * BK, dg);
      lfrag(1, as, bs, 16);
      mma(0);
      __builtin_amdgcn_sched_group_barrier(SG_DS_RD, 4 + 4 * RD2, 0);  // sub-step 0's fragments
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_amdgcn_sched_group_barrier(SG_VMEM_RD, VMS, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DS_RD, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_VMEM_RD, VMS, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DS_RD, RD2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
      }
      lfrag(0, as, bs, 32);
      mma(1);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_amdgcn_sched_group_barrier(SG_DS_RD, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DS_RD, RD2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
      }
      lfrag(1, as, bs, 48);
      mma(0);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_amdgcn_sched_group_barrier(SG_DS_RD, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DS_RD, RD2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
      }
      lstore(cur ^ 1, dg);  // that stage was last read before the previous barrier
      mma(1);
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        __builtin_amdgcn_sched_group_barrier(SG_DS_WR, WRS, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
      }
      __syncthreads();
    }
  };
  if (MODE != 2 && it.row0 == it.nrows)
    kloop(std::true_type{});
  else
    kloop(std::false_type{});

  // Epilogue.  bf16(v) of the wave's whole 128 x 128 tile goes to its own LDS
  // region (the stages are free after the last barrier) and is read back as
  // 16-byte row chunks for the normal store.  The a x / b A term is loaded
  // whole (32 x 16 B per lane) before the staging, so the wave waits for global
  // memory once.  The symmetric products' mirror and the transposed O of R > C
  // write the final values back to the staging tile and read them as 8-row
  // column chunks with the LDS transpose read.  (The mirror of B = b A + c A A
  // is the normal tile transposed: A is exactly symmetric, so is A A.)
  const bool mirror = MODE != 2 && it.row0 != it.nrows;
  const bool trout = FIN && T.ns_tr;
  const KAON_G uint16_t* eop = G((const uint16_t*)(MODE == 1 ? nb.a : xc));
  const int lde = MODE == 1 ? mp : kp;
  const bool oaln = (T.C & 7) == 0;
  if (MODE != 0) {
#pragma unroll
    for (int u = MODE == 2 ? 16 : 0; u < 32; ++u) {
      const int i = u >> 3, j = (u >> 1) & 3, q = lane + 64 * (u & 1);
      ev[u] = *(const KAON_G ku4*)(eop + (int64_t)(wr0 + i * 32 + (q >> 2)) * lde + wc0 + j * 32 + (q & 3) * 8);
    }
  }
  // acc[i][j] holds block (i, j) transposed: lane l has output row l % 32 of
  // the block, columns 8 (r / 4) + 4 (l / 32) + r % 4 -- one 8-byte LDS write
  // per 4 registers
  uint16_t* stg = lds + w * (128 * WLD);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t lo = f2bf2(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
        const uint32_t hi = f2bf2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
        *(uint64_t*)&stg[(i * 32 + (lane & 31)) * WLD + j * 32 + 8 * g + 4 * (lane >> 5)] = (uint64_t)lo | ((uint64_t)hi << 32);
      }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
  __builtin_amdgcn_wave_barrier();
  // u = (32 x 32 sub-tile i, j) x half h: rows rr = q / 4, 8 columns from c8
  bool nan = false;  // some result of this lane is NaN
#pragma unroll
  for (int u = 0; u < 32; ++u) {
    const int i = u >> 3, j = (u >> 1) & 3, q = lane + 64 * (u & 1), rr = q >> 2, c8 = (q & 3) * 8;
    const ku4 xv = *(const ku4*)&stg[(i * 32 + rr) * WLD + j * 32 + c8];
    const ku4 ov = MODE == 0 ? xv : ns_comb8<MODE>(xv, ev[u], ca, cb, cc, nan);
    if (!FIN)
      *(KAON_G ku4*)G(out + (int64_t)(wr0 + i * 32 + rr) * ldc + wc0 + j * 32 + c8) = ov;
    else if (!trout)
      ns_st8(nb.mo, T.C, wr0 + i * 32 + rr, wc0 + j * 32 + c8, (int)T.R, (int)T.C, oaln, ov);
    // each lane rewrites the chunk it read: no other lane touches it
    if (MODE != 0 && (mirror || trout)) *(ku4*)&stg[(i * 32 + rr) * WLD + j * 32 + c8] = ov;
  }
  if (FIN && __builtin_amdgcn_ballot_w64(nan) != 0) {
    // O holds torch's 0x7FC0 for every NaN: a wave that made one goes over its
    // tile again -- O's chunks recomputed (the a x term read again) and
    // rewritten, or (transposed O) the staged chunks rewritten before the
    // transposed pass reads them
    for (int u = 0; u < 32; ++u) {
      const int i = u >> 3, j = (u >> 1) & 3, q = lane + 64 * (u & 1), rr = q >> 2, c8 = (q & 3) * 8;
      ku4 ov = *(const ku4*)&stg[(i * 32 + rr) * WLD + j * 32 + c8];
      if (!trout) {
        const ku4 e = *(const KAON_G ku4*)(eop + (int64_t)(wr0 + i * 32 + rr) * lde + wc0 + j * 32 + c8);
        ov = ns_comb8<MODE>(ov, e, ca, cb, cc, nan);
      }
      ov = ku4{ns_canon2(ov.x), ns_canon2(ov.y), ns_canon2(ov.z), ns_canon2(ov.w)};
      if (trout)
        *(ku4*)&stg[(i * 32 + rr) * WLD + j * 32 + c8] = ov;
      else
        ns_st8(nb.mo, T.C, wr0 + i * 32 + rr, wc0 + j * 32 + c8, (int)T.R, (int)T.C, oaln, ov);
    }
  }
  if (!mirror && !trout) return;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  // Transposed pass: 16-lane group gq of u takes columns c0 .. c0 + 15 and
  // rows r0 .. r0 + 7 of sub-tile (i, j); lane s of the group points the
  // transpose read at row r0 + s / 4 (+ 4), columns c0 + 4 (s % 4) .. + 3, and
  // lane s receives column c0 + s, rows r0 .. r0 + 3 (r0 + 4 .. + 7): the
  // 16 bytes of row c0 + s of the transposed tile from column r0.
  const int gq = lane >> 4, sl = lane & 15;
#pragma unroll
  for (int u = 0; u < 32; ++u) {
    const int i = u >> 3, j = (u >> 1) & 3, h = u & 1;
    const int c0 = j * 32 + 16 * (gq & 1), r0 = i * 32 + 8 * ((gq >> 1) + 2 * h);
    const uint16_t* p = stg + (r0 + (sl >> 2)) * WLD + c0 + 4 * (sl & 3);
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p + 4 * WLD));
    const ku4 mv = __builtin_bit_cast(ku4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    if (mirror)
      *(KAON_G ku4*)G(out + (int64_t)(wc0 + c0 + sl) * ldc + wr0 + r0) = mv;
    else
      ns_st8(nb.mo, T.C, wc0 + c0 + sl, wr0 + r0, (int)T.R, (int)T.C, oaln, mv);
  }
}

// 8 consecutive bf16 of a row-major matrix from column c of row r; zeros
// outside rows x cols.  ALN: the row stride is a multiple of 8 (every chunk is
// 16-byte aligned).
__device__ __forceinline__ ku4 ns_ld8(const uint16_t* p, int64_t ld, int r, int c, int rows, int cols, bool aln) {
  if (r >= rows) return ku4{0u, 0u, 0u, 0u};
  const KAON_G uint16_t* q = G(p) + (int64_t)r * ld + c;
  if (aln && c + 8 <= cols) return *(const KAON_G ku4*)q;
  uint32_t h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = c + e < cols ? (uint32_t)q[e] : 0u;
  return ku4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

// x = bf16(v / den) on 8 packed bf16 (torch's bf16 division: fp32 quotient,
// rounded to bf16; a NaN stays some NaN, made 0x7FC0 when O is written)
__device__ __forceinline__ ku4 ns_scale8(ku4 v, double rden) {
  auto two = [&](uint32_t w) {
    return f2bf2(div_r64(__uint_as_float(w << 16), rden), div_r64(__uint_as_float(w & 0xFFFF0000u), rden));
  };
  return ku4{two(v.x), two(v.y), two(v.z), two(v.w)};
}

// The transposed iterate of an R > C matrix, x(r0 + i, c0 + j) = bf16(M(c0 + j,
// r0 + i) / den), in 128 x 128 tiles; elements outside M's rows x cols read as
// 0 (the iterate's zero padding).  The iterate's rows are a multiple of 128
// long, so its writes are 16-byte and in range.  A tile goes through an LDS
// tile of M's rows (256 bytes each) whose 16-byte chunks are XOR-swizzled by
// 2 (row % 4), and comes back as 8-row column chunks by the LDS transpose read:
// lane s of a 16-lane group points at tile row 8 g + s / 4 (+ 4), columns
// 16 ci + 4 (s % 4) .. + 3, and receives column 16 ci + s, rows 8 g .. 8 g + 7
// -- the 16 bytes of x row r0 + 16 ci + s from column c0 + 8 g.  The four rows
// of a read sit in four different 32-byte bank groups.
struct NsTrTile {
  const uint16_t* m;
  int64_t ldm;
  int rows, cols;
  uint16_t* x;
  int64_t ldx;
  double rden;
};
constexpr int NS_NQ = TILE * TILE / 8 / 256;  // 16-byte chunks per thread per tile

// source rows c0 .. c0 + 127 (tile rows), columns r0 .. r0 + 127
__device__ __forceinline__ void ns_tr_load(const NsTrTile& a, int r0, int c0, ku4 (&v)[NS_NQ]) {
  const bool ma = (a.ldm & 7) == 0;
#pragma unroll
  for (int s = 0; s < NS_NQ; ++s) {
    const int q = threadIdx.x + 256 * s, tt = q >> 4, ch = q & 15;
    v[s] = ns_ld8(a.m, a.ldm, c0 + tt, r0 + ch * 8, a.rows, a.cols, ma);
  }
}

__device__ __forceinline__ void ns_tr_stage(const ku4 (&v)[NS_NQ], uint16_t* tile) {
#pragma unroll
  for (int s = 0; s < NS_NQ; ++s) {
    const int q = threadIdx.x + 256 * s, tt = q >> 4, ch = q & 15;
    *(ku4*)&tile[tt * TILE + ((ch ^ (2 * (tt & 3))) << 3)] = v[s];
  }
}

__device__ __forceinline__ void ns_tr_store(const NsTrTile& a, int r0, int c0, const uint16_t* tile) {
  // wave w, step k: column block ci of 16 x rows, 8-column groups g = 4 gh + (lane / 16)
  const int tid = threadIdx.x, w = tid >> 6, gq = (tid >> 4) & 3, sl = tid & 15;
#pragma unroll
  for (int k = 0; k < NS_NQ; ++k) {
    const int P = k * 4 + w, ci = P & 7, g = 4 * (P >> 3) + gq;
    const int row = 8 * g + (sl >> 2), ch = (2 * ci + ((sl & 3) >> 1)) ^ (2 * (row & 3));
    const uint16_t* p = tile + row * TILE + (ch << 3) + 4 * (sl & 1);
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p + 4 * TILE));
    const ku4 t = __builtin_bit_cast(ku4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    *(KAON_G ku4*)G(a.x + (int64_t)(r0 + 16 * ci + sl) * a.ldx + c0 + 8 * g) = ns_scale8(t, a.rden);
  }
}

// Rows [r0, r1) of the iterate over its whole width, x = bf16(M / den) with
// zeros past M's rows x cols: whole rows of M and of x are long contiguous
// runs.  A thread takes every 256th 16-byte chunk of the rows, four at a time
// with their loads issued first.
__device__ __forceinline__ void ns_prep_rows(const uint16_t* m, int64_t ldm, int rows, int cols, uint16_t* x,
                                             int64_t ldx, int r0, int r1, double rden) {
  const bool ma = (ldm & 7) == 0;
  const int nch = (int)(ldx >> 3);  // 16-byte chunks per row of x
  const int dr = 256 / nch, dc = 256 % nch;
  int r = r0 + (int)threadIdx.x / nch, c = (int)threadIdx.x % nch;
  while (r < r1) {
    ku4 v[4];
    int rs[4], cs[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      rs[u] = r;
      cs[u] = c;
      v[u] = r < r1 ? ns_ld8(m, ldm, r, c * 8, rows, cols, ma) : ku4{0u, 0u, 0u, 0u};
      r += dr;
      c += dc;
      if (c >= nch) {
        c -= nch;
        ++r;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (rs[u] < r1) *(KAON_G ku4*)G(x + (int64_t)rs[u] * ldx + cs[u] * 8) = ns_scale8(v[u], rden);
  }
}

// x = bf16(M / den) into the padded iterate (transposed when R > C), zeros in
// the padding; den = bf16(bf16(||M||) + 1e-7) from the workspace (phase 8).
// Transposed: one item = one tile (kind 0) or 2 x 2 tiles (kind 1, a big-tile
// item).  Otherwise the tk items of a row tile split its rows: item (a, b)
// takes rows [a T + b T / tk, a T + (b + 1) T / tk) over the whole width.
__global__ __launch_bounds__(256) void k_ns_prep(const KaonTensor* __restrict__ D,
                                                 const KaonItem* __restrict__ items, float* ws) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[TILE * TILE];
  const KaonItem it = items[blockIdx.x];
  if (it.tensor < 0) return;  // an idle big-tile item
  const KaonTensor& T = D[it.tensor];
  const NsBufs nb = ns_bufs(ws, T);
  const double rden = rcp64(G(ws)[T.ws_scal + 2]);
  if (!T.ns_tr) {
    const int tt = it.kind ? 2 * TILE : TILE, tk = T.k_pad / tt;
    const int r0 = it.row0 * tt + it.nrows * tt / tk, r1 = it.row0 * tt + (it.nrows + 1) * tt / tk;
    ns_prep_rows(nb.mo, T.C, (int)T.R, (int)T.C, nb.x0, T.k_pad, r0, r1, rden);
    return;
  }
  // the sub * sub tiles of the item, the next tile's loads issued before the
  // current one is staged
  const NsTrTile a{nb.mo, T.C, (int)T.R, (int)T.C, nb.x0, T.k_pad, rden};
  const int sub = it.kind ? 2 : 1, ntile = sub * sub;
  ku4 v[NS_NQ], vn[NS_NQ];
  ns_tr_load(a, it.row0 * sub * TILE, it.nrows * sub * TILE, v);
  for (int s = 0; s < ntile; ++s) {
    const int i0 = (it.row0 * sub + s / sub) * TILE, t0 = (it.nrows * sub + s % sub) * TILE;
    if (s) __syncthreads();  // the previous tile's transpose reads are done
    ns_tr_stage(v, tile);
    if (s + 1 < ntile)
      ns_tr_load(a, (it.row0 * sub + (s + 1) / sub) * TILE, (it.nrows * sub + (s + 1) % sub) * TILE, vn);
    __syncthreads();
    ns_tr_store(a, i0, t0, tile);
#pragma unroll
    for (int q = 0; q < NS_NQ; ++q) v[q] = vn[q];
  }
}

int ns_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  kaon_set_error(std::string(what) + ": " + hipGetErrorString(e));
  return (int)e;
}

}  // namespace

int kaon_ns_run(const KaonLaunch& L, int steps, hipStream_t st) {
  if (L.n_ns_rect <= 0) return 0;
  if (steps < 1) {
    kaon_set_error("kaon_adamuon: ns_steps must be >= 1");
    return -1;
  }
  float* ws = (float*)L.workspace;
  const float a = 3.4445f, b = -4.7750f, c = 2.0315f;  // adamuon.py:106
  hipLaunchKernelGGL(k_ns_prep, dim3(L.n_ns_rect), dim3(256), 0, st, L.descs, L.ns_rect_items, ws);
  int rc = ns_check("kaon: Newton-Schulz input launch");
  // big-tile items lead both lists
  const int nsq_b = L.n_ns_sq_big, nrect_b = L.n_ns_rect_big;
  const int nsq_s = L.n_ns_sq - nsq_b, nrect_s = L.n_ns_rect - nrect_b;
  if (nsq_b < 0 || nrect_b < 0 || nsq_s < 0 || nrect_s < 0) {
    kaon_set_error("kaon_adamuon: inconsistent Newton-Schulz item counts");
    return -1;
  }
  const KaonItem* sq_s = L.ns_sq_items + nsq_b;
  const KaonItem* rect_s = L.ns_rect_items + nrect_b;
  for (int s = 0; s < steps && !rc; ++s) {
    const int par = s & 1;
    if (nsq_b) hipLaunchKernelGGL(k_ns_gemm2<0>, dim3(nsq_b), dim3(256), 0, st, L.descs, L.ns_sq_items, ws, par, a, b, c);
    if (nsq_s) hipLaunchKernelGGL(k_ns_gemm<0>, dim3(nsq_s), dim3(256), 0, st, L.descs, sq_s, ws, par, a, b, c);
    if (nsq_b) hipLaunchKernelGGL(k_ns_gemm2<1>, dim3(nsq_b), dim3(256), 0, st, L.descs, L.ns_sq_items, ws, par, a, b, c);
    if (nsq_s) hipLaunchKernelGGL(k_ns_gemm<1>, dim3(nsq_s), dim3(256), 0, st, L.descs, sq_s, ws, par, a, b, c);
    // the last iteration writes O over M
    const bool fin = s == steps - 1;
    if (nrect_b && fin)
      hipLaunchKernelGGL((k_ns_gemm2<2, true>), dim3(nrect_b), dim3(256), 0, st, L.descs, L.ns_rect_items, ws, par,
                         a, b, c);
    else if (nrect_b)
      hipLaunchKernelGGL(k_ns_gemm2<2>, dim3(nrect_b), dim3(256), 0, st, L.descs, L.ns_rect_items, ws, par, a, b, c);
    if (nrect_s && fin)
      hipLaunchKernelGGL((k_ns_gemm<2, true>), dim3(nrect_s), dim3(256), 0, st, L.descs, rect_s, ws, par, a, b, c);
    else if (nrect_s)
      hipLaunchKernelGGL(k_ns_gemm<2>, dim3(nrect_s), dim3(256), 0, st, L.descs, rect_s, ws, par, a, b, c);
    rc = ns_check("kaon: Newton-Schulz GEMM launch");
  }
  return rc;
}
