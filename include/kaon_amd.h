/*
 * kaon_amd.h -- C ABI of the MI355X (gfx950) fused optimizer-step library.
 *
 * This is the drop-in boundary for the optimizer-step hot path of
 * K-Optimizers ("kaon" 0.7.4).  The reference is pure Python: its only
 * operator boundary for this path is the Triton launch sequence behind
 * `Adakaon(fused=True)` (src/kaon/adakaon.py:387-738 launching
 * src/kaon/_fused_triton.py kernels with int64 device pointer arrays
 * g_addr/p_addr/m_addr/mscale_addr/row_addr/col_addr, int32 Rs/Cs, fp32
 * scalars lr/beta1/beta2/eps1/clip/wd and the SR seed, plus constexpr flags
 * LOWP/MOM/CAUTIOUS/WD/GC/SR -- _fused_triton.py:1183-1245, adakaon.py:
 * 506-513, 533-539), and MSAM's 4-bit perturbation launch
 * (src/kaon/msam.py:238-290 -> _fused_triton.py:1145-1179).  Lion
 * (src/kaon/lion.py:322-485) and AdaMuon (src/kaon/adamuon.py:327-615) call
 * torch ops directly; this ABI covers all four optimizers, AdaPNM
 * (src/kaon/adapnm.py, whose Triton path _fused_triton.py:724-1143 is launched
 * from adapnm.py:647-980) and KProdigy's two passes (src/kaon/kprodigy.py:306-441,
 * 744-960).
 *
 * Conventions
 *  - Plain C types only.  Every pointer inside KaonTensor / KaonItem points to
 *    device memory owned by the caller (torch); the library never allocates.
 *  - Every entry point returns 0 on success or a non-zero status; the text of
 *    the last error is available from kaon_last_error() (thread-local).
 *  - Launches are asynchronous on the caller's HIP stream (hipStream_t passed
 *    as void*); no entry point synchronizes the host.
 *  - bf16 tensors are 16-bit patterns (uint16), fp32 tensors are float.
 */
#ifndef KAON_AMD_H
#define KAON_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KAON_ABI_VERSION 10

/* element types of params / grads (p.dtype, p.grad.dtype); fp16 params and
 * grads (both fp16) step in Adakaon, Lion, AdaMuon and AdaPNM plans only,
 * written by RN or kahan */
enum { KAON_F32 = 0, KAON_BF16 = 1, KAON_F16 = 2 };

/* momentum storage ("momentum_dtype"), _momentum_codec.py:253-406 */
enum { KAON_MOM_NONE = 0, KAON_MOM_F32 = 1, KAON_MOM_BF16 = 2, KAON_MOM_INT8 = 3, KAON_MOM_4BIT = 4 };

/* low-precision weight write ("bf16_method"), _backend.py:82-98; fp32
 * params always take the plain fp32 subtraction */
enum { KAON_SR = 0, KAON_RN = 1, KAON_KAHAN = 2 };

/* optimizer selected by a plan / step */
enum { KAON_OPT_ADAKAON = 0, KAON_OPT_LION = 1, KAON_OPT_ADAMUON = 2, KAON_OPT_ADAPNM = 3, KAON_OPT_KPRODIGY = 4 };

/* per-launch flags (KaonHyper.flags) */
enum {
  KAON_F_GC = 1,        /* gradient centralization (_backend.py:147-177) */
  KAON_F_CAUTIOUS = 2,  /* cautious masking (_backend.py:127-142) */
  KAON_F_WD = 4,        /* weight_decay != 0 */
  KAON_F_EPS = 8,       /* eps1 > 0 adds eps1 to g^2 (_factored.py:35-39) */
  KAON_F_MOMENTUM = 16, /* beta1 > 0 and a momentum buffer exists */
  KAON_F_NK_REMOVE = 32,/* Nekaon: remove the previous climb first (msam.py:386-388) */
  KAON_F_NK_CLIMB = 64, /* Nekaon: climb along the new momentum (msam.py:395-403) */
  KAON_F_SRC_O = 128,   /* set by the library for AdaMuon's factored passes: the row kernels
                           read the orthogonalized O from the workspace instead of the grad */
  KAON_F_PNM = 256,     /* set by the library for AdaPNM: the 1-D second moment is
                           v*beta2 + (1-beta2)*g*g (adapnm.py:1243-1244) */
  KAON_F_AMS = 512,     /* AdaPNM ams_bound: 1-D denominators from the running max of v */
  KAON_F_PD_COUPLED = 1024, /* KProdigy pass 1: weight decay folded into the gradient
                               (decouple=False, kprodigy.py:342-349) */
  KAON_F_PD_STATS = 2048,   /* KProdigy pass 1: update s and the D statistics this step */
  KAON_F_GC_WRITE = 4096,   /* Adakaon / Lion apply and KProdigy pass 2: also store the
                               centralized gradient over p.grad of the tensors whose
                               gc_write is set, as the reference's native path leaves it
                               (centralize_grads_, _backend.py:147-177) */
  KAON_F_TORCH_ORDER = 8192, /* Adakaon / Lion steps and kaon_momentum_sumsq: the step's fp32
                               sums in torch CPU's order instead of the canonical 64-lane one
                               (below): the GC row means (_backend.py:147-177), the factored
                               row / column means and the row factors' mean (_factored.py:48-52,
                               76-82), the RMS clip norm (_backend.py:45-47), MSAM's per-tensor
                               momentum norm (msam.py:219-221) */
  KAON_F_PD_BLOCKFAC = 16384 /* KProdigy pass 1: some tensor of the plan has fb_r > 0 (its
                                second moment factored over its last two dims) */
};

/*
 * One parameter of the multi-tensor launch (the descriptor table entry that
 * replaces the reference's per-role pointer arrays).  Layout: the param and
 * grad are viewed as a row-major [R, C] matrix -- R = shape[0], C = numel/R
 * for ndim >= 2 (conv weights matrixized, adakaon.py:975-981), R = 1 and
 * C = numel for 1-D params.  State tensors are the reference's own state
 * entries (adakaon.py:318-335, lion.py:210-241, _momentum_codec.py:293-361).
 */
typedef struct KaonTensor {
  const void* g;          /* grad [R*C], g_dtype (never written) */
  void* p;                /* param [R*C], p_dtype, updated in place */
  void* m;                /* momentum codes/values (layout by codec), in place */
  float* m_scale;         /* int8: [R] per-row (1 for 1-D); 4-bit: [nblocks] */
  float* row;             /* factored: "row" [R] */
  float* col;             /* factored: "col" [C] */
  float* v;               /* 1-D: "v" [C] */
  void* shift;            /* kahan compensation [R*C] in p_dtype */
  void* m2;               /* AdaPNM: "m_neg", layout as m ("m_pos"); adapnm.py:451-500 */
  float* m2_scale;        /* AdaPNM: "m_neg_scale" */
  float* max_v;           /* AdaPNM ams_bound, 1-D: "max_v" [C] */
  float* pd_s;            /* KProdigy: "s" [pd_ns] */
  const float* pd_p0;     /* KProdigy: "p0" [pd_ns], or its single 0.0 when pd_p0_scalar */
  int64_t pd_ns;          /* KProdigy: ceil(n / pd_slice), the sliced length */
  int32_t pd_slice;       /* KProdigy: slice_p */
  int32_t pd_p0_scalar;   /* KProdigy: "p0" is the 0-dim zero (the initial slice had norm 0) */
  int32_t full_v;         /* KProdigy: per-element second moment "v" on a matrix (second_moment
                             "full"); 1-D KProdigy tensors always set it */
  int32_t by_size;        /* set by kaon_plan: descs[k].by_size is the tensor that per-tensor
                             workgroup k takes, the tensors by decreasing numel (longest first) */
  const uint16_t* noise[3]; /* optional injected SR noise per stream (tests) */
  int64_t R, C;           /* matrixized shape */
  int64_t n;              /* R * C */
  /* workspace offsets, in 4-byte words from the workspace base (kaon_plan) */
  int64_t ws_row;         /* 5 arrays of R words: mu, rf, rs, amax, oldscale */
  int64_t ws_col;         /* cf [C] */
  int64_t ws_part;        /* column partials [2][ngroups][C], one row per run: of q = g^2 (+eps1)
                             and, for the RMS clip, of g^2 / row */
  int64_t ws_blk;         /* 4-bit: 2 arrays of nblocks words: amax, oldscale */
  int64_t ws_scal;        /* 5 + ceil(C / KAON_COLITEM) words (6 for 1-D): clip divisor, keep
                             count, KProdigy num / den (MSAM / AdaMuon norms), mean(row), then
                             the clip's partial sums, one per finalize item */
  int64_t ws_aux;         /* AdaMuon: Newton-Schulz buffers, bf16: M then O [R*C], the iterate
                             X and its successor [m_pad*k_pad] each, A and B [m_pad^2] each;
                             KProdigy: the D statistics' block sums, [2][ceil(pd_ns / KAON_FLAT_ITEM)] */
  int32_t tensor_id;      /* SR counter field: index in the optimizer's param list */
  int32_t block4;         /* 4-bit block size (m_block) */
  int32_t factored;       /* ndim >= 2 */
  int32_t ngroups;        /* number of runs (column partials) */
  float sqrt_n;           /* (float)sqrt((double)n), the rms divisor (_backend.py:45-47) */
  int32_t vec_rows;       /* 16-byte vector path for row chunks (C % 8 == 0 or one row, aligned) */
  int32_t vec_flat;       /* 16-byte vector path for flat chunks (all bases aligned) */
  int32_t ns_tr;          /* AdaMuon: Newton-Schulz iterates on the transpose (R > C) */
  int32_t m_pad, k_pad;   /* AdaMuon: min(R,C) and max(R,C) rounded up to the tile (KAON_NS_TILE,
                             or twice that for big matrices) */
  int32_t fast_lanes;     /* set by kaon_plan: lanes per row of the phase-5/6 fast kernel (8..64) */
  int32_t gc_write;       /* under KAON_F_GC_WRITE: 1 = store this tensor's centralized gradient
                             over g, 0 = leave g as given (the reference's fused Adakaon
                             centralizes p.grad in place only for the params it routes to its
                             native path, adakaon.py:396-401, 448-468) */
  int32_t fb_r, fb_c;     /* KProdigy factor_conv_as_matrix=False on a tensor of 3+ dims: the
                             second moment is factored over its last two dims, blocks of
                             [fb_r, fb_c] elements ("row" [n / fb_c], "col" [n / fb_r],
                             kprodigy.py:286-288); 0 = the [R, C] factoring */
} KaonTensor;

/* A work item.  Runs and slices: rows [row0, row0 + nrows) of tensor
 * `tensor`, kind = rows per wave group (RW); a slice is at most 4 * RW rows, a
 * run at most KAON_RUN slices.  Finalize items: kind 0 = columns [row0, row0+nrows),
 * kind 1 = row statistics.  Flat items: elements [row0, row0 + nrows).
 * Newton-Schulz tiles: row0 = tile row, nrows = tile column of the padded
 * matrices, kind = 0 for KAON_NS_TILE tiles, 1 for 2 * KAON_NS_TILE tiles (the
 * symmetric products list only row <= column for those).  The big tiles are
 * interleaved per XCD (item KAON_NS_XCDS * i + x is XCD x's i-th) and include
 * idle items, tensor = -1, where one XCD's list is shorter than another's. */
typedef struct KaonItem {
  int32_t tensor;
  int32_t row0;
  int32_t nrows;
  int32_t kind;
} KaonItem;

/* torch CPU's order (KAON_F_TORCH_ORDER), as torch 2.10 on x86-64 computes the
 * reference's sums (aten/src/ATen/native/cpu/SumKernel.cpp, the norm kernel):
 * a row's sum takes 8-float vectors, four side by side, in a cascade of four
 * levels whose first takes 2^max(4, ceil(log2(rows))/4) rows of 32 floats, then
 * the leftover vectors, the four slots, the scalar tail and the 8 lanes in
 * order; a column's sum is the same cascade down the rows (blocks of 32
 * columns; the rest of the columns four row slots apiece); ||U|| keeps 8 lanes,
 * lane k a sequential fused multiply-add chain over elements k, k+8, ..., the
 * lanes added in order, then the tail.  The chain has no parallel form, so the
 * clip costs n/8 dependent fma per tensor in this mode.
 *
 * Work decomposition and canonical reduction order shared with the CPU
 * oracle.  Row sums: 64 lanes, lane l adds the 8-element chunks l, l+64, ...
 * in order, then an xor butterfly.  Column sums: wave groups of
 * RW = max(1, KAON_ROW_BUDGET / chunks-per-lane) consecutive rows (summed in
 * row order), slices of 4 wave groups (folded in order), runs of KAON_RUN
 * slices (added in order, one column partial per run), runs added in order.
 * A slice is one pass of a workgroup of 4 wave64; a run is one workgroup. */
#define KAON_ROW_BUDGET 20
#define KAON_RUN 4
/* Columns per column-finalize work item. */
#define KAON_COLITEM 2048

/* Row classes of the slice kernels (KaonPlanInfo.row_runs). */
#define KAON_ROW_CLASSES 7
/* Tile edge of the Newton-Schulz GEMMs; the iterate is zero-padded to it. */
#define KAON_NS_TILE 128
/* XCDs of the target GPU (MI355X: 8 of 32 CUs, each with its own L2): the
 * big Newton-Schulz tiles are laid out for a launch's workgroup b running on
 * XCD b % KAON_NS_XCDS. */
#define KAON_NS_XCDS 8

/*
 * Host-side plan: kaon_plan() fills the workspace offsets of every
 * descriptor and the work-item arrays.  The caller uploads descriptors and
 * items to device memory and allocates `ws_words * 4` bytes of workspace.
 */
typedef struct KaonPlanInfo {
  int32_t n_tensors;
  int32_t n_row_items;    /* runs, sorted by phase-1 register class (row_items) */
  int32_t n_fin_items;    /* finalize items (phase 2) */
  int32_t n_flat_items;   /* flat items of KAON_FLAT_ITEM elements (MSAM perturbation) */
  int32_t row_runs[KAON_ROW_CLASSES]; /* runs per row class, in row_items order: classes 0-2
                             bf16 grads with 16-byte rows of <= 4, 10, 24 chunks per lane
                             (prefetching kernels); 3-5 other rows of <= 4, 10, 24 chunks
                             held in registers; 6 streamed rows */
  int32_t n_fast;         /* items at the head of elem_items that take the specialized kernels */
  int32_t n_elem_items;   /* phase-5/6 items (elem_items) */
  int32_t n_ns_sq;        /* AdaMuon: tiles of the m_pad x m_pad products (ns_sq_items) */
  int32_t n_ns_rect;      /* AdaMuon: tiles of the m_pad x k_pad iterate (ns_rect_items) */
  int32_t n_ns_sq_big;    /* of which the leading big-tile items (kind 1) */
  int32_t n_ns_rect_big;
  int64_t ws_words;       /* workspace size in 4-byte words */
  /* The tensors whose torch-order clip norm is long (descs[k].by_size for k <
   * n_long; see kaon_adakaon_step): their chains run on a second stream beside
   * the other tensors' clip, keep count and apply.  Their phase-5/6 items are the
   * leading n_long_fast of the specialized items and the leading n_long_rest of
   * the others (elem_items[n_fast ..)).  n_long = 0: one stream. */
  int32_t n_long, n_long_fast, n_long_rest;
  int32_t reserved;
} KaonPlanInfo;

/* What a plan is built for (one param group and dtype pair). */
typedef struct KaonPlanArgs {
  int32_t opt;            /* KAON_OPT_* */
  int32_t codec;          /* KAON_MOM_* of the group (KAON_MOM_NONE without momentum) */
  int32_t p_dtype, g_dtype;
  int32_t bf16_method;    /* KAON_SR / KAON_RN / KAON_KAHAN */
} KaonPlanArgs;

/* Elements per flat work item. */
#define KAON_FLAT_ITEM 16384

/* Device-side tables of one planned group, passed to every step entry point. */
typedef struct KaonLaunch {
  const KaonTensor* descs;    /* device copy of the planned descriptors */
  const KaonItem* row_items;  /* device: runs by register class (phases 1, 3, AdaMuon momentum) */
  const KaonItem* elem_items; /* device: phase-5/6 items, specialized-kernel ones first */
  const KaonItem* fin_items;  /* device */
  const KaonItem* flat_items; /* device */
  const KaonItem* ns_sq_items;   /* device, AdaMuon */
  const KaonItem* ns_rect_items; /* device, AdaMuon */
  int32_t n_tensors, n_row_items, n_fin_items, n_flat_items;
  int32_t row_runs[KAON_ROW_CLASSES];
  /* n_fast: the leading elem_items that take the specialized phase-5/6 kernel;
   * a caller may lower it to 0 to send every item to the generic kernel (same
   * results, bit for bit; the GPU tests use this to check the two kernels) */
  int32_t n_fast, n_elem_items;
  int32_t n_ns_sq, n_ns_rect;
  int32_t n_ns_sq_big, n_ns_rect_big;
  void* workspace;            /* device, ws_words * 4 bytes, 16-byte aligned */
  int64_t ws_words;           /* KaonPlanInfo.ws_words of the plan that filled descs: the
                                 workspace the descriptors' offsets address, in 4-byte words */
  int32_t n_long, n_long_fast, n_long_rest; /* KaonPlanInfo's (0, or n_fast lowered below
                                 n_long_fast: the torch-order step on one stream) */
  int32_t reserved;
} KaonLaunch;

/* Per-launch hyper-parameters of one param group, rounded to fp32 on the
 * host exactly as the reference's torch ops see them (python float ->
 * fp32 scalar):  w1 = 1 - beta1, w2 = 1 - beta2 (lerp weights), wdl = lr*wd
 * (Adakaon/AdaMuon, adakaon.py:1007-1009) or wd (Lion, lion.py:476-477).
 * AdaPNM (_coeffs, adapnm.py:998-1016; step t = the group's step count after
 * its increment): lr = lr / (1 - beta1^t); b1 = beta1^2, a1 = 1 - beta1^2;
 * b2 = beta2, a2 = w2 = 1 - beta2; eps1 = eps; wdl = 1 - lr*wd (the decoupled
 * decay multiplier, :1231-1232); pn_pos = 1 + beta0, pn_neg = -beta0,
 * pn_rnorm = 1 / sqrt((1+beta0)^2 + beta0^2); bc2 = sqrt(1 - beta2^t);
 * clip 0 = no clip. */
typedef struct KaonHyper {
  float lr;               /* Adakaon/Lion lr; AdaMuon passes 0.2*lr (adamuon.py:88, 588) */
  float w1, w2;
  float eps1;
  float wdl;
  float clip;
  float b1, b2, a1, a2;   /* Lion: beta1, beta2, 1-beta1, 1-beta2 */
  float nk_k;             /* Nekaon k (rho = -k), nekaon.py:162-171 */
  float nk_bound_old;     /* frozen climb bound of the previous climb (msam.py:169-188) */
  float nk_bound_new;     /* |k| * clip * lr at this climb */
  float pn_pos, pn_neg, pn_rnorm, bc2; /* AdaPNM */
  /* KProdigy (kprodigy.py:306-386, 723-808; b1 = beta1, w1 = 1 - beta1, b2 = beta2,
   * w2 = 1 - beta2, eps1 = eps_factored, wdl = wd for the pass-1 coupled decay):
   * pd_tg = d*(1 - beta1), pd_vval = d*d*(1 - beta2), pd_alpha_s, pd_beta3 of the s EMA,
   * pd_d = d before this step's D update (the momentum's d), pd_dn = d after it,
   * pd_floor = dn*eps, pd_cap = 1/(dn*eps) (pass 2), pd_dlr = dlr of the old d, pd_wdl =
   * wd*dlr (decoupled decay) */
  float pd_tg, pd_vval, pd_alpha_s, pd_beta3, pd_d, pd_dn, pd_floor, pd_cap, pd_dlr, pd_wdl;
  int32_t flags;          /* KAON_F_* */
  int32_t p_dtype, g_dtype, codec, bf16_method;
  int32_t ns_steps;       /* AdaMuon Newton-Schulz iterations */
  uint32_t step;          /* SR key word 1 (the optimizer step count) */
  uint64_t seed;          /* SR key word 0 (low 32 bits used) */
} KaonHyper;

int kaon_abi_version(void);
const char* kaon_last_error(void);

/* Plan a launch group (the host half of the descriptor table; replaces the
 * pointer-array caches PointerArrayCache / OneDimPointerCache,
 * _fused_triton.py:1183-1320).  descs: host array of n descriptors with
 * pointers, shapes, block4 and tensor_id filled; on return their ws_*,
 * ngroups, sqrt_n, vec_* and fast_lanes fields are set.  row_items holds
 * n_row_items runs; elem_items holds n_elem_items phase-5/6 items: slices for
 * the generic kernel, and for the specialized kernel slices of 4 * kind rows
 * whose kind (rows per wave) is a multiple of 64 / fast_lanes.
 * Item arrays may be NULL to query sizes; info is
 * always filled.  Tensors may hold up to 2^32 - 1 elements; from 2^31 on only
 * 2-D tensors of Adakaon and Lion plans (Nekaon and MSAM plan as Adakaon).
 * Returns 0, or non-zero with kaon_last_error() set (e.g. a tensor of 2^32 or
 * more elements, or a momentum codec without its buffer). */
int kaon_plan(const KaonPlanArgs* args, KaonTensor* descs, int32_t n, KaonItem* row_items,
              KaonItem* elem_items, KaonItem* fin_items, KaonItem* flat_items, KaonItem* ns_sq_items,
              KaonItem* ns_rect_items, KaonPlanInfo* info);

/* Adakaon step over one planned param group, Nekaon's remove/climb fused in
 * when the KAON_F_NK_* flags are set.  Replaces Adakaon._fused_step and the
 * native per-param/foreach step (adakaon.py:339-409, 793-1014) and MSAM.step's
 * remove/climb around it (msam.py:375-406). */
int kaon_adakaon_step(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* Size of the static workspace of kaon_adakaon_step_noalloc, per device. */
#define KAON_NOALLOC_WS_BYTES (32u * 1024u * 1024u)

/* kaon_adakaon_step without the caller's workspace: the same kernels and
 * results, with the workspace taken from a device array of
 * KAON_NOALLOC_WS_BYTES that the library holds on every device it runs on
 * until the process ends (L->workspace is ignored).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The size checked is the launch's own L->ws_words (the plan's
 * KaonPlanInfo.ws_words): a launch that needs more than
 * KAON_NOALLOC_WS_BYTES / 4 words, or that carries no size, is rejected with
 * an error before anything is enqueued.  Allocates nothing.  Every call on a
 * device shares that device's array, so calls that overlap on one device (two
 * streams or two host threads) race; the device the stream belongs to must be
 * current. */
int kaon_adakaon_step_noalloc(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* Lion step over one planned param group (lion.py:322-352, 416-485). */
int kaon_lion_step(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* AdaMuon step over one planned group of 2-D / conv params (plan opt =
 * KAON_OPT_ADAMUON): momentum of the raw grad, Newton-Schulz quintic
 * iteration as bf16 MFMA GEMMs, factored second moment of the orthogonal
 * factor, clip, 0.2*lr scale (hp->lr carries 0.2*lr), WD, cautious against
 * the grad, write.  Replaces AdaMuon._step_one_param / _factored_bucket and
 * zeropower_via_newtonschulz5(_stacked) (adamuon.py:97-149, 434-501,
 * 557-593).  1-D params take an Adakaon plan with hp->lr = 0.2*lr
 * (adamuon.py:594-604). */
int kaon_adamuon_step(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* AdaPNM step over one planned param group (plan opt = KAON_OPT_ADAPNM):
 * decoupled WD, factored (or 1-D, optionally AMSBound) second moment with
 * bias correction, EMA of this step's positive momentum with the raw grad
 * (decay beta1^2), positive-negative mix, RMS clip, lr / (1 - beta1^t),
 * cautious against the grad, write.  m is "m_pos" and m2 "m_neg": odd steps
 * (hp->step) take m as the positive buffer, even steps m2
 * (_pos_neg_prefixes, adapnm.py:588-596).  Replaces AdaPNM._step_one_param /
 * _factored_bucket / _nonfactored_bucket (adapnm.py:1069-1275) and the fused
 * launches of adapnm.py:647-980. */
int kaon_adapnm_step(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* KProdigy over one planned param group (plan opt = KAON_OPT_KPRODIGY).  Pass 1:
 * the factored row/col EMAs (second_moment "factored"), the GC row means, the
 * first moment of d*g in its codec and the full v, and when KAON_F_PD_STATS is
 * set the s EMA and each tensor's D statistics num = FSUM(g (p0 - p)) and den =
 * FSUM(|s|) over its sliced elements (FSUM: blocks of KAON_FLAT_ITEM elements in
 * the 64-lane order, then the 64-lane order over the blocks), left in the
 * tensor's scalar words 2 and 3 of the workspace.  The caller folds them over
 * every tensor of the D scope in param order and updates D as
 * KProdigy._step_scope does (kprodigy.py:355-380).  Pass 2: the update with the
 * new d and the old dlr (kprodigy.py:383-386, 768-808): cautious count, then the
 * apply (int8 / 4-bit momenta are requantized here, as pass 1's absmax left them).
 * Replaces KProdigy._pass1_per_param / _pass1_foreach and _update_one_param /
 * _update_foreach (kprodigy.py:392-441, 443-674, 744-960). */
int kaon_kprodigy_pass1(const KaonLaunch* L, const KaonHyper* hp, void* stream);
int kaon_kprodigy_pass2(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* The same steps restricted to the phases whose bit is set in `mask`
 * (bit k = phase k: 1 row statistics, 2 column/row finalize, 3 clip sums,
 * 4 clip divisor, 5 keep-count + momentum absmax, 6 apply; Lion uses 1, 5,
 * 6).  For
 * profiling one kernel at a time; running all phases in order is the step.
 * No counterpart in the reference, which has no phase boundary to expose. */
int kaon_adakaon_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream);
int kaon_lion_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream);
/* AdaMuon: bit 8 = momentum pass, norm and Newton-Schulz input; bit 9 =
 * Newton-Schulz GEMMs and the orthogonal factor O; then bits 1-6 as above on
 * O.  The step is mask 0x37E. */
int kaon_adamuon_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream);
/* AdaPNM: bits 1-6; phase 3 also records the new positive momentum's int8 row /
 * 4-bit block absmax, phase 5 is the cautious keep count. */
int kaon_adapnm_phases(const KaonLaunch* L, const KaonHyper* hp, uint32_t mask, void* stream);

/* MSAM norm="none" perturbation p += clamp(nan_to_num(factor * dequant(m)), +-bound)
 * (msam.py:202-235; fused 4-bit twin _fused_triton.py:1145-1179), used by
 * Nekaon.eval()/train() (msam.py:294-311).  stream_id selects the SR noise
 * stream (0 = removal, 2 = climb). */
int kaon_msam_apply(const KaonLaunch* L, const KaonHyper* hp, float factor, float bound,
                    uint32_t stream_id, void* stream);

/* MSAM norm="tensor" perturbation (msam.py:219-222, 231-235): each tensor's
 * p += m * s with its own s = reciprocal(||m|| + eps) * signed_rho (torch's
 * python-scalar-over-tensor division), ||m|| the fp32 square root of the sum
 * kaon_momentum_sumsq stored for the tensor, which must run first on the same
 * launch.  stream_id as for kaon_msam_apply. */
int kaon_msam_apply_tensor(const KaonLaunch* L, const KaonHyper* hp, float signed_rho, float eps,
                           uint32_t stream_id, void* stream);

/* Each tensor's sum of squares of its dequantized momentum into its scalar word
 * 2 of the workspace (rows in the 64-lane order, then the rows in that order),
 * for MSAM norm="global", whose climb is rho * m / (||m|| + eps) with ||m|| over
 * every momentum of the net (_global_mnorm, msam.py:191-199; the caller adds
 * the tensors in param order in fp32 and takes the fp32 square root).  The
 * climb and its removal then run through kaon_msam_apply with that factor and
 * an infinite bound. */
int kaon_momentum_sumsq(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* Leaves p.grad centralized, as the reference's native path does
 * (centralize_grads_, _backend.py:147-177, called at adakaon.py:352-353 and
 * :399-401): after a step with KAON_F_GC, every 2-D / conv gradient of the plan
 * is overwritten with round(g - mu) in its dtype, mu the row means the step
 * used.  The step itself never writes the gradient; callers that mirror the
 * reference's fused path (which centralizes in-kernel, adakaon.py:387-409) skip
 * this call. */
int kaon_gc_writeback(const KaonLaunch* L, const KaonHyper* hp, void* stream);

/* ---------------------------------------------------------- primitives */
/* _quant_int8 (_momentum_codec.py:72-83): rows x cols fp32 -> int8 codes +
 * per-row scale (rows = 1 for a 1-D tensor). */
int kaon_quant_int8(const float* m, int64_t rows, int64_t cols, int8_t* q, float* scale, void* stream);
/* _quant_4bit (_momentum_codec.py:122-141): n fp32 -> packed nibbles + per-block scale. */
int kaon_quant_4bit(const float* m, int64_t n, int32_t block, uint8_t* packed, float* scale,
                    void* stream);
/* dequant of int8 ([rows, cols], per-row scale) or 4-bit (flat blocks) codes to fp32. */
int kaon_dequant(int32_t codec, const void* m, const float* scale, int64_t rows, int64_t cols,
                 int32_t block, float* out, void* stream);
/* _add_stochastic_bf16_ bit trick (_stochastic_rounding.py:70-103) with explicit noise. */
int kaon_sr_round(const float* x, const uint16_t* noise, int64_t n, uint16_t* out, void* stream);
/* Philox4x32-10 SR noise words of (seed, step, tensor id, stream) for elements [0, n). */
int kaon_sr_noise(uint16_t* out, int64_t n, uint64_t seed, uint32_t step, uint32_t tensor_id,
                  uint32_t stream_id, void* stream);
/* Streaming copy (bytes must be a multiple of 16, both pointers 16-B aligned): the
 * measured HBM read+write ceiling the step is compared against. */
int kaon_copy(const void* src, void* dst, int64_t bytes, void* stream);
/* The apply's access mix as a measured ceiling: per element read 2 B of bf16 g,
 * 2 B of bf16 p and 1 B of int8 m, write p and m back (5:3 read:write, 8 B per
 * element, n % 8 == 0).  No counterpart in the reference: it bounds what the
 * phase-6 apply (the same streams plus its arithmetic) can reach on the device. */
int kaon_apply_ceiling(const void* g, void* p, void* m, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KAON_AMD_H */
