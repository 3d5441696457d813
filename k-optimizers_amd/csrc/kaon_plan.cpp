// kaon_plan.cpp -- host half of the multi-tensor descriptor table.
//
// The reference rebuilds int64 device pointer arrays per role (g, p, m,
// m_scale, row, col) and int32 shape arrays for every fused launch, cached per
// param set (PointerArrayCache / OneDimPointerCache,
// src/kaon/_fused_triton.py:1183-1320; built at adakaon.py:489-539, 623-738).
// Here one descriptor per tensor carries every pointer and shape, and the plan
// adds what the HIP kernels need: a workspace layout for the per-row /
// per-column / per-block intermediates and three work-item tables.
//   runs        KAON_RUN slices of 4 wave groups of RW consecutive rows of
//               one tensor (RW = max(1, 20 / chunks-per-lane); the whole
//               tensor for a 1-D param), sorted by register class (row
//               length, grad dtype) so each class is one launch with a fixed
//               register budget;
//   elem items  phase-5/6 slices; those of the specialized kernel round RW up
//               to a multiple of the rows it works on at once;
//   fin items   KAON_COLITEM columns of one factored tensor, or its row stats;
//   flat items  KAON_FLAT_ITEM consecutive elements of one tensor (the MSAM
//               perturbation).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "kaon_amd.h"

// Error text reported by kaon_last_error() (defined with the kernels).
void kaon_set_error(const std::string& s);

namespace {
int plan_fail(const std::string& s) {
  kaon_set_error(s);
  return -1;
}

bool aligned(const void* p, uintptr_t a) { return p == nullptr || ((uintptr_t)p % a) == 0; }

int64_t round4(int64_t x) { return (x + 3) & ~int64_t(3); }

int64_t chunks_per_lane(int64_t C) {
  const int64_t nch = (C + 7) / 8;
  const int64_t cpl = (nch + 63) / 64;
  return cpl < 1 ? 1 : cpl;
}

// rows per wave group (the column-sum order of the CPU oracle)
int64_t rows_per_wave(int64_t C) {
  const int64_t rw = KAON_ROW_BUDGET / chunks_per_lane(C);
  return rw < 1 ? 1 : rw;
}

// Lanes per row of the specialized phase-5/6 kernel: a power of two in
// [max(8, G), 64] (G = 4-bit lanes per block) whose rounds of chunks cover the
// row's C/8 chunks with the fewest idle lanes (ties: more lanes).  A wave
// then works on 64/L rows at a time.
int32_t fast_lanes(int64_t C, int64_t gl) {
  const int64_t nfull = C / 8;
  int32_t best = 64;
  double best_use = 0.0;
  for (int32_t L = 64; L >= 8 && L >= gl; L >>= 1) {
    const double use = (double)nfull / (double)(L * ((nfull + L - 1) / L));
    if (use > best_use + 1e-12) {
      best_use = use;
      best = L;
    }
  }
  return best;
}

// row class of a slice (phase 1, AdaPNM's phase 3): 0-2 bf16 grads in
// 16-byte rows of <= 4, 10, 24 chunks per lane, loaded whole into registers
// by the prefetching kernels; 3-5 other rows held in registers up to 4, 10
// and 24 chunks per lane (24 only for bf16 grads); 6 streamed rows
int row_class(const KaonTensor& t, int32_t g_dtype) {
  if (!t.factored) return 6;
  const int64_t cpl = chunks_per_lane(t.C);
  if (g_dtype == KAON_BF16 && t.vec_rows && t.C % 8 == 0 && cpl <= 24) return cpl <= 4 ? 0 : cpl <= 10 ? 1 : 2;
  if (cpl <= 4) return 3;
  if (cpl <= 10) return 4;
  if (cpl <= 24 && g_dtype == KAON_BF16) return 5;
  return 6;
}
}  // namespace

// Tensors whose slices take the specialized phase-5/6 kernels: bf16 params and
// grads, stochastic rounding, factored, 16-byte aligned rows, and for 4-bit
// momentum blocks of 8*G elements (G | 64): whole chunks, inside rows or across them.
bool fast_eligible(const KaonPlanArgs& a, const KaonTensor& t) {
  if (a.opt == KAON_OPT_KPRODIGY) return false;
  if (a.p_dtype != KAON_BF16 || a.g_dtype != KAON_BF16 || a.bf16_method != KAON_SR) return false;
  if (!t.factored || !t.vec_rows || t.C % 8 != 0) return false;
  if (a.codec == KAON_MOM_F32) return false;
  // the specialized kernel addresses bf16 elements by 32-bit byte offsets
  if (t.n > (int64_t(1) << 31)) return false;
  if (a.codec == KAON_MOM_4BIT) {
    const int64_t B = t.block4;
    if (B % 8 != 0 || B / 8 > 64 || 64 % (B / 8) != 0) return false;
  }
  return true;
}

// The big Newton-Schulz tiles in the order the GPU runs them.  Workgroup b of a
// launch runs on XCD b % KAON_NS_XCDS, and each XCD starts its own workgroups in
// order, so item KAON_NS_XCDS * i + x is XCD x's i-th tile.  A matrix's tiles go
// to one XCD and share its L2 (a matrix with more than 1/64 of the launch's work
// is cut into pieces of at most that much).  Pieces are dealt with the longest
// tiles first, each to the XCD with the least work so far; an XCD's list that
// comes out shorter than the longest ends in idle items (tensor -1).  A tile
// costs its K length: k_pad + m_pad for the products (x x^T, then A A), m_pad
// for the iterate (B x).
static void ns_xcd_order(std::vector<KaonItem>& v, const KaonTensor* descs, bool sq) {
  constexpr int X = KAON_NS_XCDS;
  if (v.empty()) return;
  auto cost = [&](const KaonItem& it) {
    const KaonTensor& t = descs[it.tensor];
    return sq ? (int64_t)t.k_pad + t.m_pad : (int64_t)t.m_pad;
  };
  int64_t total = 0;
  for (const KaonItem& it : v) total += cost(it);
  const int64_t cap = std::max<int64_t>(1, total / (8 * X));
  struct Piece {
    size_t b, e;
    int64_t c, per;
  };
  std::vector<Piece> pieces;
  for (size_t i = 0; i < v.size();) {
    const int64_t per = cost(v[i]);
    size_t j = i;
    int64_t c = 0;
    while (j < v.size() && v[j].tensor == v[i].tensor && (j == i || c + per <= cap)) {
      c += per;
      ++j;
    }
    pieces.push_back(Piece{i, j, c, per});
    i = j;
  }
  std::stable_sort(pieces.begin(), pieces.end(), [](const Piece& a, const Piece& b) {
    return a.per != b.per ? a.per > b.per : a.c > b.c;
  });
  std::vector<std::vector<KaonItem>> lists(X);
  int64_t load[X] = {};
  for (const Piece& pc : pieces) {
    const int x = (int)(std::min_element(load, load + X) - load);
    load[x] += pc.c;
    lists[x].insert(lists[x].end(), v.begin() + pc.b, v.begin() + pc.e);
  }
  size_t len = 0;
  for (const auto& l : lists) len = std::max(len, l.size());
  std::vector<KaonItem> out(len * X, KaonItem{-1, 0, 0, 1});
  for (int x = 0; x < X; ++x)
    for (size_t i = 0; i < lists[x].size(); ++i) out[i * X + x] = lists[x][i];
  v.swap(out);
}

// Words of AdaMuon's Newton-Schulz block (bf16 buffers, each 16-byte aligned):
// M / O [R*C], the iterate and its successor [m_pad*k_pad], A and B [m_pad^2].
int64_t ns_words(const KaonTensor& t) {
  const int64_t rc = round4((t.R * t.C + 1) / 2);
  const int64_t x = round4((int64_t)t.m_pad * t.k_pad / 2);
  const int64_t a = round4((int64_t)t.m_pad * t.m_pad / 2);
  return rc + 2 * x + 2 * a;
}

extern "C" int kaon_plan(const KaonPlanArgs* args, KaonTensor* descs, int32_t n, KaonItem* row_items,
                         KaonItem* elem_items, KaonItem* fin_items, KaonItem* flat_items, KaonItem* ns_sq_items,
                         KaonItem* ns_rect_items, KaonPlanInfo* info) {
  if (!info) return plan_fail("kaon_plan: info is NULL");
  if (!args) return plan_fail("kaon_plan: args is NULL");
  const int32_t opt = args->opt, codec = args->codec, g_dtype = args->g_dtype;
  if (n < 0 || (n > 0 && !descs)) return plan_fail("kaon_plan: bad descriptor array");
  if (opt != KAON_OPT_ADAKAON && opt != KAON_OPT_LION && opt != KAON_OPT_ADAMUON && opt != KAON_OPT_ADAPNM &&
      opt != KAON_OPT_KPRODIGY)
    return plan_fail("kaon_plan: unknown optimizer");
  if (codec < KAON_MOM_NONE || codec > KAON_MOM_4BIT) return plan_fail("kaon_plan: unknown codec");
  if (g_dtype != KAON_F32 && g_dtype != KAON_BF16 && g_dtype != KAON_F16)
    return plan_fail("kaon_plan: unknown grad dtype");
  if (args->p_dtype != KAON_F32 && args->p_dtype != KAON_BF16 && args->p_dtype != KAON_F16)
    return plan_fail("kaon_plan: unknown param dtype");
  if (g_dtype == KAON_F16 || args->p_dtype == KAON_F16) {
    // fp16 params (RN or kahan writes, _backend.py:82-98) with fp16 grads, on the
    // generic kernels of Adakaon, Lion, AdaMuon, AdaPNM and KProdigy
    if (opt != KAON_OPT_ADAKAON && opt != KAON_OPT_LION && opt != KAON_OPT_ADAMUON && opt != KAON_OPT_ADAPNM &&
        opt != KAON_OPT_KPRODIGY)
      return plan_fail("kaon_plan: fp16 params step in Adakaon, Lion, AdaMuon, AdaPNM and KProdigy plans only");
    if (g_dtype != KAON_F16 || args->p_dtype != KAON_F16) return plan_fail("kaon_plan: fp16 params take fp16 grads");
  }
  std::memset(info, 0, sizeof(*info));
  info->n_tensors = n;

  int64_t off = 0;
  struct RowIt {
    KaonItem it;
    int cls;
    int64_t size;
    bool fast;
  };
  std::vector<RowIt> rows, elems;
  std::vector<KaonItem> fins, flats, ns_sq, ns_rect, ns_sq_big, ns_rect_big;
  // the row kernels of an AdaMuon plan read the bf16 orthogonal factor
  const int32_t row_dtype = opt == KAON_OPT_ADAMUON ? (int32_t)KAON_BF16 : g_dtype;
  for (int32_t i = 0; i < n; ++i) {
    KaonTensor& t = descs[i];
    if (t.R < 1 || t.C < 0) return plan_fail("kaon_plan: tensor " + std::to_string(i) + " has a bad shape");
    t.n = t.R * t.C;
    // Element offsets inside a tensor are 32-bit unsigned in the generic
    // phase-5/6, MSAM and momentum-norm kernels: up to 2^32 - 1 elements.
    // From 2^31 on only 2-D tensors of Adakaon / Lion plans (Nekaon and MSAM
    // step through Adakaon's) are planned; the other optimizers' kernels and
    // the 1-D row path keep signed 32-bit offsets.
    if (t.n >= (int64_t)1 << 32)
      return plan_fail("kaon_plan: tensor " + std::to_string(i) + " has >= 2^32 elements");
    if (t.n >= (int64_t)1 << 31 && (!t.factored || (opt != KAON_OPT_ADAKAON && opt != KAON_OPT_LION)))
      return plan_fail("kaon_plan: tensor " + std::to_string(i) +
                       " has >= 2^31 elements; tensors that large step only as 2-D params of "
                       "Adakaon / Lion / Nekaon / MSAM");
    if (!t.factored && t.R != 1) return plan_fail("kaon_plan: a 1-D tensor must have R == 1");
    if (opt == KAON_OPT_ADAMUON && !t.factored)
      return plan_fail("kaon_plan: tensor " + std::to_string(i) +
                       " is 1-D; AdaMuon plans take 2-D / conv params (1-D params step through an Adakaon "
                       "plan with lr scaled by 0.2)");
    if (codec == KAON_MOM_4BIT && t.block4 < 1) return plan_fail("kaon_plan: 4-bit block size must be >= 1");
    if (codec != KAON_MOM_NONE && t.R * t.C > 0 && !t.m)
      return plan_fail("kaon_plan: tensor " + std::to_string(i) + " has no momentum buffer for the planned codec");
    if ((codec == KAON_MOM_INT8 || codec == KAON_MOM_4BIT) && t.R * t.C > 0 && !t.m_scale)
      return plan_fail("kaon_plan: tensor " + std::to_string(i) + " has no momentum scales for the planned codec");
    t.sqrt_n = (float)std::sqrt((double)(t.n > 1 ? t.n : 1));
    const int64_t rw = rows_per_wave(t.C);
    const int64_t slice_rows = 4 * rw;
    const int64_t run_rows = KAON_RUN * slice_rows;
    t.ngroups = (int32_t)((t.R + run_rows - 1) / run_rows);
    if (opt == KAON_OPT_KPRODIGY) {
      if (!t.factored && !t.full_v)
        return plan_fail("kaon_plan: KProdigy 1-D tensor " + std::to_string(i) + " needs full_v (a per-element v)");
      if (t.pd_slice < 1) return plan_fail("kaon_plan: KProdigy slice_p must be >= 1");
      if (t.pd_ns != (t.R * t.C + t.pd_slice - 1) / t.pd_slice)
        return plan_fail("kaon_plan: KProdigy tensor " + std::to_string(i) + " has pd_ns != ceil(n / slice_p)");
      if (t.R * t.C > 0 && (!t.pd_s || !t.pd_p0))
        return plan_fail("kaon_plan: KProdigy tensor " + std::to_string(i) + " needs s and p0");
      if (t.fb_r != 0 || t.fb_c != 0) {
        // factored over the last two dims: whole blocks inside each matrixized row
        if (t.fb_r < 1 || t.fb_c < 1 || t.full_v || !t.factored || t.C % ((int64_t)t.fb_r * t.fb_c) != 0)
          return plan_fail("kaon_plan: KProdigy tensor " + std::to_string(i) +
                           " has a bad block factoring (fb_r x fb_c must divide its rows)");
      }
    } else {
      t.full_v = 0;
      t.fb_r = t.fb_c = 0;
    }
    if (opt == KAON_OPT_ADAPNM && (!t.m || !t.m2))
      return plan_fail("kaon_plan: AdaPNM tensor " + std::to_string(i) + " needs both momentum buffers (m, m2)");
    const bool al = aligned(t.g, 16) && aligned(t.p, 16) && aligned(t.m, 16) && aligned(t.v, 16) &&
                    aligned(t.shift, 16) && aligned(t.row, 16) && aligned(t.col, 16) && aligned(t.m2, 16) &&
                    aligned(t.max_v, 16) && aligned(t.pd_s, 16) && (t.pd_p0_scalar || aligned(t.pd_p0, 16));
    t.vec_flat = al ? 1 : 0;
    t.vec_rows = (al && (t.C % 8 == 0 || t.R == 1)) ? 1 : 0;
    // workspace: 4-word aligned arrays
    t.ws_row = off;
    off = round4(off + 5 * t.R);
    t.ws_col = off;
    t.ws_part = off;
    if (t.fb_r > 0) {
      // block factoring: the blocks' column factors [n / fb_r], then their row factors [n / fb_c]
      off = round4(off + t.n / t.fb_r);
      t.ws_part = off;
      off = round4(off + t.n / t.fb_c);
    } else if (t.factored && !t.full_v) {
      off = round4(off + t.C);
      t.ws_part = off;
      // the column partials of G^2 and, after them, of the clip's G^2 / row
      off = round4(off + 2 * (int64_t)t.ngroups * t.C);
    }
    t.ws_blk = off;
    if (codec == KAON_MOM_4BIT) {
      const int64_t nb = (t.n + t.block4 - 1) / t.block4;
      off = round4(off + 2 * nb);
    }
    // scalar words: the clip divisor, the keep count, two of KProdigy's / MSAM's,
    // and the clip's algebraic sum: rm, then one partial per finalize item (or one)
    t.ws_scal = off;
    off = round4(off + 5 + (t.factored ? (t.C + KAON_COLITEM - 1) / KAON_COLITEM : 1));
    t.ws_aux = off;
    t.ns_tr = 0;
    t.m_pad = t.k_pad = 0;
    if (opt == KAON_OPT_ADAMUON) {
      const int64_t m = std::min(t.R, t.C), k = std::max(t.R, t.C);
      t.ns_tr = t.R > t.C ? 1 : 0;
      // Matrices of at least 4 * KAON_NS_TILE rows take 2 * KAON_NS_TILE tiles
      // when the padding that adds grows the m^2 terms by at most 1.5x: the
      // big-tile kernel runs at more than twice the small one's rate (m = 640
      // pads to 768, m = 320 stays on small tiles).
      const int64_t m128 = (m + KAON_NS_TILE - 1) / KAON_NS_TILE * KAON_NS_TILE;
      const int64_t m256 = (m + 2 * KAON_NS_TILE - 1) / (2 * KAON_NS_TILE) * (2 * KAON_NS_TILE);
      const bool big = m128 >= 4 * KAON_NS_TILE && 2 * m256 * m256 <= 3 * m128 * m128;
      const int64_t tile = big ? 2 * KAON_NS_TILE : KAON_NS_TILE;
      t.m_pad = (int32_t)((m + tile - 1) / tile * tile);
      t.k_pad = (int32_t)((k + tile - 1) / tile * tile);
      off += ns_words(t);
      if (t.n > 0) {
        const int32_t tm = (int32_t)(t.m_pad / tile), tk = (int32_t)(t.k_pad / tile);
        // A = x x^T and B = b A + c A A are symmetric: big tiles cover a <= b
        // only, their mirror is written with them
        for (int32_t a = 0; a < tm; ++a)
          for (int32_t b = big ? a : 0; b < tm; ++b) (big ? ns_sq_big : ns_sq).push_back(KaonItem{i, a, b, big});
        // big tiles of the iterate column by column: the tiles of one column
        // read the same columns of x
        if (big) {
          for (int32_t b = 0; b < tk; ++b)
            for (int32_t a = 0; a < tm; ++a) ns_rect_big.push_back(KaonItem{i, a, b, 1});
        } else {
          for (int32_t a = 0; a < tm; ++a)
            for (int32_t b = 0; b < tk; ++b) ns_rect.push_back(KaonItem{i, a, b, 0});
        }
      }
    }
    if (opt == KAON_OPT_KPRODIGY) {
      // the D statistics' block sums (num, den) per KAON_FLAT_ITEM sliced elements
      const int64_t nfb = (t.pd_ns + KAON_FLAT_ITEM - 1) / KAON_FLAT_ITEM;
      off = round4(off + 2 * nfb);
    }
    if (t.n == 0) continue;
    // runs (row items): kind = rows per wave group
    const int cls = row_class(t, row_dtype);
    const bool fast = fast_eligible(*args, t);
    for (int64_t r0 = 0; r0 < t.R; r0 += run_rows) {
      KaonItem it{i, (int32_t)r0, (int32_t)std::min<int64_t>(run_rows, t.R - r0), (int32_t)rw};
      rows.push_back({it, cls, t.n, fast});
    }
    // phase-5/6 items: the slices, except for the specialized kernel, whose
    // waves take a multiple of 64/L rows (L = fast_lanes)
    t.fast_lanes = 64;
    if (fast) {
      t.fast_lanes = fast_lanes(t.C, codec == KAON_MOM_4BIT ? t.block4 / 8 : 1);
      const int64_t per = 64 / t.fast_lanes;
      const int64_t frw = (rw + per - 1) / per * per;
      for (int64_t r0 = 0; r0 < t.R; r0 += 4 * frw) {
        KaonItem it{i, (int32_t)r0, (int32_t)std::min<int64_t>(4 * frw, t.R - r0), (int32_t)frw};
        elems.push_back({it, cls, t.n, true});
      }
    } else {
      for (int64_t r0 = 0; r0 < t.R; r0 += slice_rows) {
        KaonItem it{i, (int32_t)r0, (int32_t)std::min<int64_t>(slice_rows, t.R - r0), (int32_t)rw};
        elems.push_back({it, cls, t.n, false});
      }
    }
    // finalize items (the factored second moment of every optimizer but Lion)
    if (t.factored && !t.full_v && t.fb_r == 0 && opt != KAON_OPT_LION) {
      for (int64_t c0 = 0; c0 < t.C; c0 += KAON_COLITEM)
        fins.push_back(KaonItem{i, (int32_t)c0, (int32_t)std::min<int64_t>(KAON_COLITEM, t.C - c0), 0});
      fins.push_back(KaonItem{i, 0, (int32_t)t.R, 1});
    }
    // flat items: blocks of the elements (MSAM perturbation), or for KProdigy of
    // the sliced elements (the D statistics)
    const int64_t nflat = opt == KAON_OPT_KPRODIGY ? t.pd_ns : t.n;
    for (int64_t e0 = 0; e0 < nflat; e0 += KAON_FLAT_ITEM)
      // the element offset as 32 unsigned bits (the kernels read it back as uint32)
      flats.push_back(KaonItem{i, (int32_t)(uint32_t)e0, (int32_t)std::min<int64_t>(KAON_FLAT_ITEM, nflat - e0), 0});
  }
  // elem order: specialized-kernel slices first, each part largest tensors first
  std::stable_sort(elems.begin(), elems.end(), [](const RowIt& a, const RowIt& b) {
    if (a.fast != b.fast) return a.fast;
    return a.size > b.size;
  });
  // register classes in ascending order; inside a class the largest tensors
  // first so their long runs of items start early
  std::stable_sort(rows.begin(), rows.end(), [](const RowIt& a, const RowIt& b) {
    if (a.cls != b.cls) return a.cls < b.cls;
    return a.size > b.size;
  });
  // finalize items tallest tensors first: an item's work grows with R (its
  // column sums run down the rows), so the longest start early.  Each item
  // writes only its own columns (or its tensor's row factors) and its clip
  // partial goes to its column block's slot, so the order moves no result.
  std::stable_sort(fins.begin(), fins.end(),
                   [&](const KaonItem& a, const KaonItem& b) { return descs[a.tensor].R > descs[b.tensor].R; });
  info->n_row_items = (int32_t)rows.size();
  info->n_fast = 0;
  for (const RowIt& r : elems) info->n_fast += r.fast ? 1 : 0;
  info->n_elem_items = (int32_t)elems.size();
  if (elem_items)
    for (size_t k = 0; k < elems.size(); ++k) elem_items[k] = elems[k].it;
  info->n_fin_items = (int32_t)fins.size();
  info->n_flat_items = (int32_t)flats.size();
  for (const RowIt& r : rows) info->row_runs[r.cls]++;
  info->ws_words = off > 0 ? off : 4;
  // per-tensor launches (the torch-order clip norm) take the longest tensors first
  {
    std::vector<int32_t> ord(n);
    for (int32_t i = 0; i < n; ++i) ord[i] = i;
    std::stable_sort(ord.begin(), ord.end(), [&](int32_t a, int32_t b) { return descs[a].n > descs[b].n; });
    for (int32_t k = 0; k < n; ++k) descs[k].by_size = ord[k];
    // The torch-order clip norm of a tensor is n / 8 dependent fmas.  The tensors
    // whose chain is at least half the longest (when that is at least 2^18 steps
    // and shorter tensors remain) run their chains on a second stream while the
    // rest step (Adakaon plans: kaon_adakaon_step).  They are a prefix of by_size,
    // and their phase-5/6 items a prefix of the specialized items and of the
    // others (both sorted largest tensors first).
    const int64_t nmax = n > 0 ? descs[ord[0]].n : 0;
    if (opt == KAON_OPT_ADAKAON && nmax >= (int64_t)1 << 21) {
      const int64_t thr = (nmax + 1) / 2;
      int32_t nl = 0;
      while (nl < n && descs[ord[nl]].n >= thr) ++nl;
      if (nl < n) {
        info->n_long = nl;
        for (const RowIt& r : elems) {
          if (descs[r.it.tensor].n < thr) continue;
          if (r.fast) ++info->n_long_fast;
          else ++info->n_long_rest;
        }
      }
    }
  }
  if (row_items)
    for (size_t k = 0; k < rows.size(); ++k) row_items[k] = rows[k].it;
  if (fin_items && !fins.empty()) std::memcpy(fin_items, fins.data(), fins.size() * sizeof(KaonItem));
  if (flat_items && !flats.empty()) std::memcpy(flat_items, flats.data(), flats.size() * sizeof(KaonItem));
  // Newton-Schulz tiles: the big-tile items first
  ns_xcd_order(ns_sq_big, descs, true);
  ns_xcd_order(ns_rect_big, descs, false);
  info->n_ns_sq_big = (int32_t)ns_sq_big.size();
  info->n_ns_rect_big = (int32_t)ns_rect_big.size();
  ns_sq.insert(ns_sq.begin(), ns_sq_big.begin(), ns_sq_big.end());
  ns_rect.insert(ns_rect.begin(), ns_rect_big.begin(), ns_rect_big.end());
  info->n_ns_sq = (int32_t)ns_sq.size();
  info->n_ns_rect = (int32_t)ns_rect.size();
  if (ns_sq_items && !ns_sq.empty()) std::memcpy(ns_sq_items, ns_sq.data(), ns_sq.size() * sizeof(KaonItem));
  if (ns_rect_items && !ns_rect.empty())
    std::memcpy(ns_rect_items, ns_rect.data(), ns_rect.size() * sizeof(KaonItem));
  return 0;
}
