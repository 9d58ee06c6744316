// Backward of the fused MLM attention for gfx950 (bf16 / fp16, MFMA 16x16x32).
//
// No counterpart in the reference: its roadmap lists backpropagation
// (README.md:26-28).  What is differentiated is the forward of fmlm_attn.hip, i.e. the
// reference's attention over [cached context || main keys] (mlm_kernel_impl.py:10-62,
// 65-216, 219-390).  For one query row with key set K, values V, P = softmax(scale q K^T)
// and O = P V:
//   delta = rowsum(dO * O),  dP = dO V^T,  dS = scale * P * (dP - delta),
//   dq = dS K,  dK = dS^T q,  dV = P^T dO.
// Two kernels, no atomics, so every gradient row has exactly one writer:
//   attn_bwd_dq_kernel   one workgroup per (query tile, head, sequence), as in the
//     forward.  One pass over the key set accumulates dq^T = K^T dS^T with an online
//     softmax (running max, lazy rescale) and yields each row's log2-sum-exp, which it
//     stores with scale * delta for the next kernel.
//   attn_bwd_dkv_kernel  one workgroup per 64-key tile of a key segment (the main keys of
//     a sequence, the causal token range of a head, or a context batch), 16 keys per
//     wave.  It walks every query row that attends to those keys in steps of 64 rows
//     (32 at D >= 256) staged through LDS and accumulates dK^T = Q^T dS and
//     dV^T = dO^T P in registers.
//     Keys whose head stride is 0 (the MLA latent) are shared by all heads and take the
//     queries of every head; with MLA (V = K) both gradients land in dk.
// Layouts: every product is in the forward's transposed MFMA form, so the accumulator
// lane (j + 16g) holds rows 4g..4g+3 of column j, and the transposed operands come from
// row-major LDS tiles through ds_read_b64_tr_b16.
#include "fmlm_common.h"

#include <algorithm>
#include <mutex>

namespace fmlm {
namespace {

constexpr int kBwdNW = 4;   // waves per workgroup
constexpr int kBwdBK = 64;  // keys per dq-kernel tile
// lazy rescale of the dq kernel's online softmax: the running max moves only when a tile's
// max exceeds it by more than this (log2 units), so 2^(z - m) <= 2^8 before rounding
constexpr float kRescaleSlack = 8.0f;

template <int D>
struct BwdCfg {
  static constexpr int NT = kBwdNW * 64;
  static constexpr int KC = D / 32;               // 32-wide contraction steps over D
  static constexpr int NDB = D / 16;              // 16-wide column blocks
  static constexpr int C8 = D / 8;                // 16-byte chunks per row
  // 16-row query blocks per wave (dq kernel): two at D = 128 (each K / V fragment then
  // feeds two MFMAs); one at D >= 256 (registers) and at D <= 64, where twice the
  // workgroups balance the grid (a batch with few query tiles per slot otherwise runs a
  // nearly empty second round) and four waves fit on a SIMD
  static constexpr int QB = D == 128 ? 2 : 1;
  static constexpr int BQ = kBwdNW * QB * 16;     // query rows per dq workgroup
  // dq kernel key tiles: unpadded rows whose 16-byte chunks are swizzled by kv_swz,
  // filled by direct global->LDS loads of RPI rows per wave-wide load.  The 512-wide
  // latent (PAD) reads rows padded to D + 16 elements, one wave-wide direct load per row:
  // the swizzled addressing's per-chunk bases do not fit beside its accumulators.
  static constexpr int CPR = D / 8;               // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;            // rows per wave-wide load
  static constexpr bool PAD = D >= 512;
  static constexpr int ROWB = (PAD ? D + 16 : D) * 2;  // LDS row pitch (bytes)
  static constexpr int TILEB = kBwdBK * ROWB;
  static constexpr int NPW = kBwdBK / RPI / kBwdNW;  // wave-wide loads per tile and tensor
  static constexpr int NKB = kBwdBK / 16;
  static constexpr int NKS = kBwdBK / 32;
  // dkv kernel: 16-key blocks per wave.  Two at the 512-wide latent (one wave per SIMD);
  // one elsewhere: at D = 128 two spill, and at D <= 64 one block per wave halves the
  // work per unit (a shared context's units walk every query of the batch, so smaller
  // units balance the grid) and lets three waves share a SIMD
  static constexpr int KB = D >= 512 ? 2 : 1;
  static constexpr int DKV_KEYS = kBwdNW * 16 * KB;  // keys per dkv workgroup
  static constexpr int QS = D >= 256 ? 32 : 64;   // query rows per dkv step (32-row groups)
  // dK/dV kernel: a query step's Q and dO rows (tiles like the dq kernel's; padded rows
  // for the latent) and its lse and delta, in two buffers (the next step loads during
  // the current one's math)
  static constexpr int DKV_NBUF = 2;
  static constexpr int STEPB = QS * ROWB;
  static constexpr int DKV_SB = 2 * STEPB + 2 * QS * 4;  // bytes per step buffer
  static constexpr int DKV_LDS = DKV_NBUF * DKV_SB;
  // waves per SIMD the kernels are built for: the 512-wide latent needs more than 256
  // registers per wave, which gfx950 gives a wave (VGPRs + AGPRs) only at one wave per SIMD
  static constexpr int WPS = D >= 512 ? 1 : 2;
  static constexpr bool MLA_ONLY = D >= 512;  // the 512-wide head dim exists for the MLA latent only
  // dq kernel: two buffers per tensor (the next tile loads during the current one's
  // math) where they fit beside the other workgroups of a CU: one at D = 256, two at
  // D <= 128 and for the latent (one workgroup per CU, no V tile since V = K)
  static constexpr int DQ_NBUF = (D <= 128 || PAD) ? 2 : 1;
  static constexpr int DQ_LDS = DQ_NBUF * (MLA_ONLY ? 1 : 2) * TILEB;
  static_assert(D % 32 == 0 && D >= 32 && D <= 512, "head dim");
};

// element offset of row (sequence b, head h, position pos) in a tensor of `layout`
FMLM_DEV int64_t row_at(int layout, int b, int h, int q0, int pos, int64_t sb, int64_t sh, int64_t sn) {
  return layout == FMLM_LAYOUT_PACKED ? (int64_t)h * sh + (int64_t)(q0 + pos) * sn
                                      : (int64_t)b * sb + (int64_t)h * sh + (int64_t)pos * sn;
}

// One key segment for key head h: rows kbase + j*ksn of k (vbase + j*vsn of v), j < n;
// the gradient rows of key j are dkbase + j*dksn of dk (dvbase + j*dvsn of dv).
struct BSeg {
  const char* k;
  const char* v;
  char* dk;
  char* dv;
  int64_t kbase, vbase, ksn, vsn;
  int64_t dkbase, dvbase, dksn, dvsn;
  int n;
  // paged context: key j is row j % FMLM_PAGE_ROWS of page pages[j / FMLM_PAGE_ROWS]
  // (ids clamped to the pool), base + page * page_elems + row * sn; the gradients are
  // float32 and accumulated atomically (a page may serve several context batches)
  const int32_t* pages;
  int64_t page_elems;
  int npool, ntab;
};

// element offset of key `key` of a segment, from `base` with row stride `sn`
FMLM_DEV int64_t key_elem(const BSeg& s, int64_t base, int64_t sn, int key) {
  if (!s.pages) return base + (int64_t)key * sn;
  int pg = s.pages[min(key / FMLM_PAGE_ROWS, max(s.ntab - 1, 0))];
  pg = min(max(pg, 0), max(s.npool - 1, 0));
  return base + (int64_t)pg * s.page_elems + (int64_t)(key % FMLM_PAGE_ROWS) * sn;
}

// keys of the context segment of context batch cb (0 without context gradients), from its
// row range [c0, c1)
FMLM_DEV int ctx_seg_keys(const fmlm_attn_params& p, int c0, int c1) {
  return (p.flags & FMLM_FLAG_PREFILL) || !p.k_ctx ? 0 : max(c1 - c0, 0);
}

// context rows of context batch cb (mlm_kernel_impl.py:297-313 packed, :132-141 dense),
// given its first row c0 and key count n (ctx_range, ctx_seg_keys)
FMLM_DEV BSeg ctx_seg_at(const fmlm_attn_params& p, const fmlm_attn_grads& g, int cb, int h, int c0, int n) {
  const bool mla = p.flags & FMLM_FLAG_MLA;
  BSeg s;
  s.n = n;
  s.k = (const char*)p.k_ctx;
  s.v = (const char*)(mla ? p.k_ctx : p.v_ctx);
  s.dk = (char*)g.dk_ctx;
  s.dv = (char*)(mla ? g.dk_ctx : g.dv_ctx);
  s.pages = nullptr;
  s.page_elems = 0;
  s.npool = s.ntab = 0;
  if (p.ctx_block_table) {  // paged: rows come from the batch's pages
    s.pages = p.ctx_block_table + (int64_t)cb * p.ctx_pages_per_batch;
    s.page_elems = p.ctx_page_stride;
    s.npool = p.ctx_rows;
    s.ntab = p.ctx_pages_per_batch;
    s.kbase = s.vbase = (int64_t)h * p.c_sh;
  } else {
    s.kbase = s.vbase = (int64_t)cb * p.c_sb + (int64_t)h * p.c_sh + (int64_t)c0 * p.c_sn;
  }
  s.dkbase = s.dvbase = s.kbase;
  s.ksn = s.vsn = s.dksn = s.dvsn = p.c_sn;
  return s;
}

// main keys of sequence b (mlm_kernel_impl.py:288-293, 360-379): its own tokens, or
// with causal_query_seq_attn the packed tokens [0, cu[b+1]) (n = those of all of them
// when b < 0); si: the ranges of sequence b (b >= 0), or n = si.mainlen when b < 0
FMLM_DEV BSeg main_seg_at(const fmlm_attn_params& p, const fmlm_attn_grads& g, int b, int h, const SeqInfo& si) {
  const bool mla = p.flags & FMLM_FLAG_MLA;
  const int64_t v_sb = mla ? p.k_sb : p.v_sb, v_sh = mla ? p.k_sh : p.v_sh, v_sn = mla ? p.k_sn : p.v_sn;
  const int64_t dv_sb = mla ? g.dk_sb : g.dv_sb, dv_sh = mla ? g.dk_sh : g.dv_sh, dv_sn = mla ? g.dk_sn : g.dv_sn;
  BSeg s;
  s.pages = nullptr;
  s.page_elems = 0;
  s.npool = s.ntab = 0;
  s.k = (const char*)p.k;
  s.v = (const char*)(mla ? p.k : p.v);
  s.dk = (char*)g.dk;
  s.dv = (char*)(mla ? g.dk : g.dv);
  s.ksn = p.k_sn;
  s.vsn = v_sn;
  s.dksn = g.dk_sn;
  s.dvsn = dv_sn;
  const bool causal = (p.flags & FMLM_FLAG_CAUSAL_SEQ) && p.cu_seqlens_q;
  if (causal) {  // packed K/V: token j is row h*sh + j*sn
    s.n = si.mainlen;
    s.kbase = (int64_t)h * p.k_sh;
    s.vbase = (int64_t)h * v_sh;
    s.dkbase = (int64_t)h * g.dk_sh;
    s.dvbase = (int64_t)h * dv_sh;
    return s;
  }
  s.n = si.len;
  s.kbase = row_at(p.kv_layout, b, h, si.q0, 0, p.k_sb, p.k_sh, p.k_sn);
  s.vbase = row_at(p.kv_layout, b, h, si.q0, 0, v_sb, v_sh, v_sn);
  s.dkbase = row_at(p.kv_layout, b, h, si.q0, 0, g.dk_sb, g.dk_sh, g.dk_sn);
  s.dvbase = row_at(p.kv_layout, b, h, si.q0, 0, dv_sb, dv_sh, dv_sn);
  return s;
}

FMLM_DEV u32x4 ld16(const char* base, int64_t elem) { return *(const u32x4*)(base + elem * 2); }

// A-operand fragment of X^T (16 columns of X from column 16db, 32 rows from row0) from a
// row-major LDS tile: lane (i + 16g) receives X[row0 + 16h + 4g + e][16db + i] as element
// 4h + e, the row order of the packed B operands below.
template <typename T>
FMLM_DEV typename Mfma<T>::v8 tr_frag(const T* tile, int rs, int row0, int db, int l16, int g) {
  const T* base = tile + (row0 + g * 4 + (l16 >> 2)) * rs + db * 16 + (l16 & 3) * 4;
  const s16x4 lo = lds_read_tr16(base);
  const s16x4 hi = lds_read_tr16(base + 16 * rs);
  return __builtin_bit_cast(typename Mfma<T>::v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Fragment reads from a row-major LDS tile of head dim D (row pitch ROWB bytes): rows of
// D elements whose 16-byte chunks are swizzled by kv_swz (logical chunk c of row r in
// physical chunk c ^ kv_swz(r)), or, with PAD, rows padded to D + 16 elements.
//   row(tile, kb, kc): A operand of rows 16kb + l16, columns 32kc + 8g .. +8;
//   col(tile, ks, db): tr_frag's fragment of X^T from rows 32ks .. +32, columns 16db .. +16.
template <typename T, int D>
struct TileReader {
  typedef BwdCfg<D> C;
  typedef typename Mfma<T>::v8 v8;
  int koff[4], voff[8], l16, g;
  FMLM_DEV TileReader(int l16_, int g_) : l16(l16_), g(g_) {
    if constexpr (!C::PAD) {
      // row fragment at kb*16*ROWB + 256*(kc/4) + koff[kc%4]; tr16 fragment of rows
      // 32ks + 16h + 4g + (l16 >> 2), columns 16db + 4*(l16 & 3) .. +4 at
      // (32ks + 16h)*ROWB + 256*(db/8) + voff[db%8]
      const int ksw = kv_swz<D>(l16);
#pragma unroll
      for (int b4 = 0; b4 < 4; ++b4) koff[b4] = l16 * C::ROWB + 16 * ((4 * b4 + g) ^ ksw);
      const int vr = 4 * g + (l16 >> 2);
      const int vsw = kv_swz<D>(vr);
      const int x = (l16 & 3) >> 1;
#pragma unroll
      for (int db = 0; db < 8; ++db) voff[db] = vr * C::ROWB + 16 * ((2 * db + x) ^ vsw) + 8 * (l16 & 1);
    }
  }
  FMLM_DEV v8 row(const char* tile, int kb, int kc) const {
    if constexpr (C::PAD) {
      return *(const v8*)((const T*)tile + (kb * 16 + l16) * (C::ROWB / 2) + kc * 32 + g * 8);
    } else {
      return *(const v8*)(tile + kb * 16 * C::ROWB + 256 * (kc / 4) + koff[kc % 4]);
    }
  }
  FMLM_DEV v8 col(const char* tile, int ks, int db) const {
    if constexpr (C::PAD) {
      return tr_frag<T>((const T*)tile, C::ROWB / 2, ks * 32, db, l16, g);
    } else {
      const char* a = tile + ks * 32 * C::ROWB + 256 * (db / 8) + voff[db % 8];
      const s16x4 lo = lds_read_tr16(a);
      const s16x4 hi = lds_read_tr16(a + 16 * C::ROWB);
      return __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  }
};

// Direct global->LDS loads of an NR-row swizzled tile: rows from the wave-uniform row-0
// address src at pitch rowb bytes (rows past `last` repeat row `last`) into the tile at
// LDS byte address lds.  Wave-wide load i = wave + j*NW brings rows [i*RPI, (i+1)*RPI),
// lane l fetching logical chunk (l % CPR) ^ kv_swz(row) of row i*RPI + l/CPR into
// physical chunk l % CPR.  Nothing waits here: the caller waits (vmcnt) and meets a
// barrier before the tile is read.
template <int D, int NR>
FMLM_DEV void dma_rows(const char* src, uint32_t rowb, int last, uint32_t lds, int wave, int lane) {
  typedef BwdCfg<D> C;
  static_assert(!C::PAD && NR % (C::RPI * kBwdNW) == 0, "whole wave-wide loads per wave");
  // the lane's offsets are recomputed per call: partial tiles and steps, and row pitches
  // other than the one the pipelined kernels precompute offsets for (see dma_rows_at)
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int row0 = wave * C::RPI + ln / C::CPR;
#pragma unroll
  for (int j = 0; j < NR / (C::RPI * kBwdNW); ++j) {
    const int row = row0 + j * kBwdNW * C::RPI;
    const int i = wave + j * kBwdNW;
    const uint32_t r = (uint32_t)min(row, last);
    dma16_sbase(src, r * rowb + 16u * (uint32_t)((ln % C::CPR) ^ kv_swz<D>(row)),
                __builtin_amdgcn_readfirstlane(lds + i * 1024));
  }
}

// The loads of dma_rows with the lane's byte offsets precomputed for a whole tile (no row
// past the end): off[j] = row_j * rowb + 16 * (chunk ^ kv_swz(row_j)).
template <int D, int NR>
FMLM_DEV void dma_rows_at(const char* src, const uint32_t (&off)[NR / (BwdCfg<D>::RPI * kBwdNW)], uint32_t lds,
                          int wave) {
#pragma unroll
  for (int j = 0; j < NR / (BwdCfg<D>::RPI * kBwdNW); ++j)
    dma16_sbase(src, off[j], __builtin_amdgcn_readfirstlane(lds + (wave + j * kBwdNW) * 1024));
}
template <int D, int NR>
FMLM_DEV void dma_offsets(uint32_t rowb, int lane, int wave, uint32_t (&off)[NR / (BwdCfg<D>::RPI * kBwdNW)]) {
  typedef BwdCfg<D> C;
  const int row0 = wave * C::RPI + lane / C::CPR;
#pragma unroll
  for (int j = 0; j < NR / (C::RPI * kBwdNW); ++j) {
    const int row = row0 + j * kBwdNW * C::RPI;
    off[j] = (uint32_t)row * rowb + 16u * (uint32_t)((lane % C::CPR) ^ kv_swz<D>(row));
  }
}

// Direct global->LDS loads of NR padded rows (the 512-wide latent: one row is one
// wave-wide 16-byte load): row r from the wave-uniform row-0 address src at pitch rowb
// bytes (rows past `last` repeat row `last`) to LDS byte address lds + r * ROWB, row r by
// wave r % kBwdNW.  Nothing waits here.
template <int D, int NR>
FMLM_DEV void dma_rows_padded(const char* src, uint32_t rowb, int last, uint32_t lds, int wave, int lane) {
  typedef BwdCfg<D> C;
  static_assert(C::PAD && C::CPR == 64 && NR % kBwdNW == 0, "one wave-wide load per padded row");
#pragma unroll
  for (int j = 0; j < NR / kBwdNW; ++j) {
    const int row = __builtin_amdgcn_readfirstlane(wave + j * kBwdNW);
    const uint32_t r = (uint32_t)min(row, last);
    dma16_sbase(uniform_ptr(src + (size_t)r * rowb), 16u * (uint32_t)lane, __builtin_amdgcn_readfirstlane(lds + row * C::ROWB));
  }
}

// ---------------------------------------------------------------------------
// Unit tables.  The workspace holds, after the row statistics (2*H*total_q floats), an
// order of the sequences (B ints, see bwd_units_kernel) and three exclusive prefix sums
// of tile counts: query tiles of BQ rows per sequence in that order (B + 1), key tiles
// of DKV_KEYS rows per sequence (B + 1) and per context batch (n_ctx + 1).  A
// workgroup maps its linear unit id to (sequence or batch, tile) by binary search, so
// the grids hold only real tiles plus a bound of one per sequence / batch.
// ---------------------------------------------------------------------------
struct UnitTables {
  int32_t* perm;  // [B]: the sequence of query-table entry r
  int32_t* q;     // [B + 1], over the sequences in perm order
  int32_t* k;     // [B + 1]
  int32_t* c;     // [n_ctx + 1]
};

FMLM_DEV UnitTables unit_tables(const fmlm_attn_params& p, const fmlm_attn_grads& g) {
  UnitTables t;
  t.perm = (int32_t*)((char*)g.workspace + 2 * (int64_t)p.H * p.total_q * 4);
  t.q = t.perm + p.B;
  t.k = t.q + p.B + 1;
  t.c = t.k + p.B + 1;
  return t;
}

constexpr int kScanThreads = 1024;

// exclusive prefix sums of ceil(len / tile) over n entries, one workgroup: each thread
// sums a run of entries, the runs are scanned within each wave by lane shuffles, and each
// wave adds the totals of the waves before it (two barriers, where a scan over all
// kScanThreads partial sums took twenty)
template <typename LenFn>
FMLM_DEV void scan_tiles(int n, int tile, LenFn len, int32_t* out, int32_t* part) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (n + kScanThreads - 1) / kScanThreads;
  const int i0 = min(tid * per, n), i1 = min(i0 + per, n);
  int sum = 0;
  for (int i = i0; i < i1; ++i) sum += (max(len(i), 0) + tile - 1) / tile;
  int incl = sum;  // inclusive scan within the wave
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off);
    if (lane >= off) incl += v;
  }
  if (lane == 63) part[wave] = incl;  // wave totals
  __syncthreads();
  int run = incl - sum;
  for (int w = 0; w < wave; ++w) run += part[w];
  for (int i = i0; i < i1; ++i) {
    out[i] = run;
    run += (max(len(i), 0) + tile - 1) / tile;
  }
  if (tid == kScanThreads - 1) out[n] = run;  // the last thread's run ends at the total
  __syncthreads();  // part is rewritten by the next scan
}

// keys a query row of sequence b attends to (context, then its own or causal main keys)
FMLM_DEV int dq_keys(const fmlm_attn_params& p, int b) {
  int c0 = 0, c1 = 0;
  if (!(p.flags & FMLM_FLAG_PREFILL) && p.k_ctx) ctx_range(p, ctx_batch_of(p, b), c0, c1);
  const SeqInfo si = seq_info(p, b);
  const bool causal = (p.flags & FMLM_FLAG_CAUSAL_SEQ) && p.cu_seqlens_q;
  return max(c1 - c0, 0) + (causal ? si.mainlen : si.len);
}

// Sequences ranked by key count, largest first (ties by index), up to this many; the
// dq kernel's query table follows that order, so the workgroups dispatched last (the
// grid runs in unit order, grid_unit) are the short ones.  More sequences keep their order.
constexpr int kRankMax = 1024;

__global__ __launch_bounds__(kScanThreads) void bwd_units_kernel(const fmlm_attn_params p, const fmlm_attn_grads g,
                                                                 int bq, int bk, int n_ctx) {
  __shared__ int32_t part[kScanThreads];
  __shared__ int32_t s_keys[kRankMax], s_perm[kRankMax];
  const UnitTables t = unit_tables(p, g);
  const int tid = threadIdx.x;
  const bool ranked = p.B <= kRankMax;
  if (ranked) {
    for (int b = tid; b < p.B; b += kScanThreads) s_keys[b] = dq_keys(p, b);
    __syncthreads();
    for (int b = tid; b < p.B; b += kScanThreads) {
      const int kb = s_keys[b];
      int r = 0;
      for (int j = 0; j < p.B; ++j) r += (s_keys[j] > kb) || (s_keys[j] == kb && j < b);
      s_perm[r] = b;  // ranks are a permutation of [0, B)
    }
    __syncthreads();
  }
  for (int r = tid; r < p.B; r += kScanThreads) t.perm[r] = ranked ? s_perm[r] : r;
  scan_tiles(p.B, bq, [&](int r) { return seq_info(p, ranked ? s_perm[r] : r).len; }, t.q, part);
  scan_tiles(p.B, bk, [&](int b) { return seq_info(p, b).len; }, t.k, part);
  scan_tiles(n_ctx, bk, [&](int cb) {
    int c0, c1;
    ctx_range(p, cb, c0, c1);
    return c1 - c0;
  }, t.c, part);
}

// ---------------------------------------------------------------------------
// Grids of both kernels: (unit, head) pairs, heads fastest.  Workgroups are dispatched in
// linear order and dealt to the 8 XCDs in turn, so with a multiple of 8 heads every unit
// of a head runs on one XCD (with 12 heads, on two), and the units that read the same
// rows (a sequence's query tiles read its keys; a key segment's units read its queries)
// share that XCD's L2.  A heads-outermost grid spreads those units over all XCDs: at 16
// heads (fp16, D = 128, per-sequence contexts) it missed L2 3.4x (dq) and 2.8x (dK/dV) as
// often and the backward took 8% longer.  The units keep their order (the dq kernel's
// longest first).  The host lays the pairs out as (x, y) with at most 2^23 workgroups per
// row (x) and heads * units < 2^31.
// ---------------------------------------------------------------------------
__host__ __device__ inline unsigned dkv_heads(const fmlm_attn_params& p, int n_ctx) {
  return (p.k_sh == 0 && (n_ctx == 0 || p.c_sh == 0)) ? 1u : (unsigned)p.H;
}
// unit u and head h of this workgroup in a grid of `heads` heads
FMLM_DEV void grid_unit(unsigned heads, int& u, int& h) {
  const unsigned w = blockIdx.y * gridDim.x + blockIdx.x;
  u = (int)(w / heads);
  h = (int)(w % heads);
}

// ---------------------------------------------------------------------------
// Key units of the dK / dV kernels: unit u of key head kh (grid_unit) is a tile of
// `keys` keys, context tiles first (unit table c), then main-key tiles (per sequence from
// unit table k, or with CAUSAL tiles of the causal token range).
// ---------------------------------------------------------------------------
struct KeyUnit {
  BSeg s;
  int kh;             // key head
  int slot, j0;       // sequence / context batch, first key of the tile
  int b_lo, b_hi;     // sequences whose queries may attend to these keys
  bool is_ctx;
  bool causal_main;   // main keys of the causal token range (key j seen by b iff j < cu[b+1])
  bool shared;        // key rows shared by all heads (head stride 0)
  SeqInfo si_lo;      // ranges of sequence b_lo (b_lo < b_hi)
};

// ---------------------------------------------------------------------------
// Unit records.  bwd_records_kernel resolves every unit of both grids once per call into
// kRecInts ints, so that a workgroup reads its unit in one round trip instead of the
// chains of dependent metadata loads (binary searches over the unit tables, then the
// sequence and context ranges) that took 5-6 us per dK/dV unit.
//   query unit (dq): [0] sequence b (-1: no rows), [1] its first row, [2..5] SeqInfo of b
//     (q0, len, ctx, mainlen), [6] context batch, [7] its first row, [8] its keys
//   key unit (dK/dV): [0] kind (0: none, 1: context tile, 2: main-key tile), [1] sequence
//     or context batch, [2] first key, [3] keys of the segment, [4] the segment's first row
//     (context row or sequence start), [5] b_lo: the first sequence whose queries attend
//     to the tile (b_hi if none), [6] b_hi, [7..10] SeqInfo of b_lo
// ---------------------------------------------------------------------------
constexpr int kRecInts = 16;

// the first N ints of record r, in one round trip: every load is issued before any of
// them is used (the compiler would otherwise sink loads into the branches on field 0 and
// wait for them one after another)
template <int N>
FMLM_DEV void load_record(const int32_t* r, int (&f)[N]) {
  static_assert(N == 9 || N == 11, "record prefix");
#pragma unroll
  for (int i = 0; i < N; ++i) f[i] = ldc(r, i);
  if constexpr (N == 9)
    asm volatile("" ::"s"(f[0]), "s"(f[1]), "s"(f[2]), "s"(f[3]), "s"(f[4]), "s"(f[5]), "s"(f[6]), "s"(f[7]), "s"(f[8]));
  else
    asm volatile("" ::"s"(f[0]), "s"(f[1]), "s"(f[2]), "s"(f[3]), "s"(f[4]), "s"(f[5]), "s"(f[6]), "s"(f[7]), "s"(f[8]),
                 "s"(f[9]), "s"(f[10]));
}

FMLM_DEV SeqInfo rec_seq_info(const int* f) {
  SeqInfo si;
  si.q0 = f[0];
  si.len = f[1];
  si.ctx = f[2];
  si.mainlen = f[3];
  return si;
}

FMLM_DEV void query_record(const fmlm_attn_params& p, const fmlm_attn_grads& g, int bq, int u, int32_t (&r)[kRecInts]) {
  const UnitTables ut = unit_tables(p, g);
#pragma unroll
  for (int i = 0; i < kRecInts; ++i) r[i] = 0;
  r[0] = -1;
  if (u >= ldc(ut.q, p.B)) return;
  const int rk = find_seq(ut.q, p.B, u);  // table entry: sequences by key count, largest first
  const int b = ldc(ut.perm, rk);
  const SeqInfo si = seq_info(p, b);
  const int qpos0 = (u - ldc(ut.q, rk)) * bq;
  if (qpos0 >= si.len) return;
  const int cb = ctx_batch_of(p, b);
  int c0, c1;
  ctx_range(p, cb, c0, c1);
  r[0] = b;
  r[1] = qpos0;
  r[2] = si.q0;
  r[3] = si.len;
  r[4] = si.ctx;
  r[5] = si.mainlen;
  r[6] = cb;
  r[7] = c0;
  r[8] = ctx_seg_keys(p, c0, c1);
}

// a tile of context batch / sequence `slot` (main keys: causal_main as in KeyUnit) from
// key j0 is attended by the queries of sequence b
FMLM_DEV bool seq_attends(const fmlm_attn_params& p, bool is_ctx, bool causal_main, int slot, int j0, int b,
                          SeqInfo& si) {
  if (is_ctx && ctx_batch_of(p, b) != slot) return false;
  si = seq_info(p, b);
  return si.len > 0 && (!causal_main || si.mainlen > j0);  // causal: tokens < cu[b+1]
}

FMLM_DEV void key_record(const fmlm_attn_params& p, const fmlm_attn_grads& g, int n_ctx, int keys, bool causal,
                         int u, int32_t (&r)[kRecInts]) {
  const int32_t* cu = p.cu_seqlens_q;
  const UnitTables ut = unit_tables(p, g);
#pragma unroll
  for (int i = 0; i < kRecInts; ++i) r[i] = 0;
  const int n_main = causal ? (min(ldc(cu, p.B), p.total_q) + keys - 1) / keys : ldc(ut.k, p.B);
  const int n_cunits = n_ctx > 0 ? ldc(ut.c, n_ctx) : 0;
  int kind = 0, slot = 0, j0 = 0, n = 0, row0 = 0, b_lo = p.B, b_hi = p.B;
  if (u < n_cunits) {
    kind = 1;
    slot = find_seq(ut.c, n_ctx, u);
    j0 = (u - ldc(ut.c, slot)) * keys;
    int c0, c1;
    ctx_range(p, slot, c0, c1);
    n = ctx_seg_keys(p, c0, c1);
    row0 = c0;
    // the sequences of this context batch: with one batch per sequence and no context
    // index, sequence `slot` alone (ctx_batch_of), else any of them
    const bool own = !p.ctx_index && p.ctx_batch > 1;
    b_lo = own ? min(slot, p.B) : 0;
    b_hi = own ? min(slot + 1, p.B) : p.B;
  } else if (u - n_cunits < n_main) {
    kind = 2;
    const int um = u - n_cunits;
    if (causal) {
      j0 = um * keys;
      n = min(ldc(cu, p.B), p.total_q);
      b_lo = j0 < n ? find_seq(cu, p.B, j0) : p.B;
    } else {
      slot = find_seq(ut.k, p.B, um);
      j0 = (um - ldc(ut.k, slot)) * keys;
      const SeqInfo si = seq_info(p, slot);
      n = si.len;
      row0 = si.q0;
      b_lo = slot;
      b_hi = slot + 1;
    }
  }
  if (kind == 0 || j0 >= n) return;
  SeqInfo si{};
  int b = b_lo;
  for (; b < b_hi; ++b)
    if (seq_attends(p, kind == 1, causal && kind == 2, slot, j0, b, si)) break;
  r[0] = kind;
  r[1] = slot;
  r[2] = j0;
  r[3] = n;
  r[4] = row0;
  r[5] = b;
  r[6] = b_hi;
  if (b < b_hi) {
    r[7] = si.q0;
    r[8] = si.len;
    r[9] = si.ctx;
    r[10] = si.mainlen;
  }
}

// one thread per unit of either grid
__global__ __launch_bounds__(256) void bwd_records_kernel(const fmlm_attn_params p, const fmlm_attn_grads g, int bq,
                                                          int bk, int n_ctx, int32_t* qrec, int nq, int32_t* krec,
                                                          int nk) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  int32_t r[kRecInts];
  if (i < nq) {
    query_record(p, g, bq, i, r);
    int4* d = (int4*)(qrec + (int64_t)i * kRecInts);
#pragma unroll
    for (int j = 0; j < kRecInts / 4; ++j) d[j] = make_int4(r[4 * j], r[4 * j + 1], r[4 * j + 2], r[4 * j + 3]);
  }
  if (i < nk) {
    key_record(p, g, n_ctx, bk, (p.flags & FMLM_FLAG_CAUSAL_SEQ) != 0, i, r);
    int4* d = (int4*)(krec + (int64_t)i * kRecInts);
#pragma unroll
    for (int j = 0; j < kRecInts / 4; ++j) d[j] = make_int4(r[4 * j], r[4 * j + 1], r[4 * j + 2], r[4 * j + 3]);
  }
}

// unit u of key head kh (grid_unit) from its record (krec: nk records); false for a
// workgroup without keys (past the units, an empty tile, or a shared segment's other heads)
template <bool CAUSAL>
FMLM_DEV bool resolve_key_unit(const fmlm_attn_params& p, const fmlm_attn_grads& g, int n_ctx, const int32_t* krec,
                               int nk, KeyUnit& k) {
  int u, kh;
  grid_unit(dkv_heads(p, n_ctx), u, kh);
  k.kh = kh;
  if (u >= nk) return false;
  int f[11];
  load_record(krec + (int64_t)u * kRecInts, f);
  const int kind = f[0];
  if (kind == 0) return false;
  k.is_ctx = kind == 1;
  k.slot = f[1];
  k.j0 = f[2];
  const int n = f[3], row0 = f[4];
  k.b_lo = f[5];
  k.b_hi = f[6];
  k.si_lo = rec_seq_info(f + 7);
  k.causal_main = CAUSAL && !k.is_ctx;
  if (k.is_ctx) {
    k.s = ctx_seg_at(p, g, k.slot, kh, row0, n);
    k.shared = p.c_sh == 0;
  } else {
    SeqInfo sm{};
    sm.q0 = row0;
    sm.len = sm.mainlen = n;
    k.s = main_seg_at(p, g, CAUSAL ? -1 : k.slot, kh, sm);
    k.shared = p.k_sh == 0;
  }
  return !(k.shared && kh > 0);  // the grid covers the larger segment kind
}

// Query steps of a key unit: (head hq, sequence b, rows [p0, p0 + qs)) over every
// sequence whose queries attend to the unit's keys, heads outermost; hq == hq_hi ends.
struct QStep {
  int hq, b, p0;
};
struct QuerySteps {
  const fmlm_attn_params* p;
  const KeyUnit* k;
  int hq_hi, qs;
  FMLM_DEV bool seq_ok(int b) const {
    SeqInfo si;
    return seq_attends(*p, k->is_ctx, k->causal_main, k->slot, k->j0, b, si);
  }
  FMLM_DEV QStep first_from(int hq, int b) const {
    while (hq < hq_hi) {
      for (; b < k->b_hi; ++b)
        if (seq_ok(b)) return QStep{hq, b, 0};
      ++hq;
      b = k->b_lo;
    }
    return QStep{hq_hi, k->b_lo, 0};
  }
  FMLM_DEV QStep next(const QStep& st) const { return next(st, seq_info(*p, st.b).len); }
  // the same, given the length of st's sequence
  FMLM_DEV QStep next(const QStep& st, int len) const {
    if (st.p0 + qs < len) return QStep{st.hq, st.b, st.p0 + qs};
    return first_from(st.hq, st.b + 1);
  }
};

// ---------------------------------------------------------------------------
// dq kernel: grid (query-tile units, H), kBwdNW waves, QB blocks of 16 rows per wave.
// LSE: the forward stored each row's log2-sum-exp (p.lse), so P = 2^(z - lse) needs no
// running max, no row sum and no rescale.
// ---------------------------------------------------------------------------
template <typename T, int D, bool LSE>
__global__ __launch_bounds__(kBwdNW * 64, BwdCfg<D>::WPS) void attn_bwd_dq_kernel(const fmlm_attn_params p,
                                                                     const fmlm_attn_grads g,
                                                                     const int32_t* qrec, int nq) {
  typedef BwdCfg<D> C;
  typedef typename Mfma<T>::v8 v8;
  constexpr int QB = C::QB;
  extern __shared__ __align__(16) char smem_raw[];

  int u, h;
  grid_unit((unsigned)p.H, u, h);
  if (u >= nq) return;
  int rec[9];  // the unit's record (query_record)
  load_record(qrec + (int64_t)u * kRecInts, rec);
  const int b = rec[0];
  if (b < 0) return;
  const int qpos0 = rec[1];
  const SeqInfo si = rec_seq_info(rec + 2);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, gq = lane >> 4;
  const float c = p.scale * kLog2e;  // scores in log2 units
  // MLA: V is K, so the K tile serves both products and no V tile is loaded
  const bool kv_same = C::MLA_ONLY || (p.flags & FMLM_FLAG_MLA);
  // software-pipelined tile (below) for the double-buffered unpadded tiles
  constexpr bool PIPE = !C::PAD && C::DQ_NBUF == 2;

  const BSeg sc = ctx_seg_at(p, g, rec[6], h, rec[7], rec[8]);  // context, then main keys
  const BSeg sm = main_seg_at(p, g, b, h, si);
  const int nt0 = (sc.n + kBwdBK - 1) / kBwdBK;
  const int nt = nt0 + (sm.n + kBwdBK - 1) / kBwdBK;

  // Q and dO fragments (B operands): lane (q + 16g), block qb, step kc holds row q's
  // columns kc*32 + 8g .. +8; delta = rowsum(dO * O) of the lane's row
  v8 qf[QB][C::KC], df[QB][C::KC];
  float delta[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = qpos0 + (wave * QB + qb) * 16 + l16;
    const bool ok = row < si.len;
    const int64_t qo = row_at(p.q_layout, b, h, si.q0, row, p.q_sb, p.q_sh, p.q_sn);
    const int64_t doo = row_at(p.o_layout, b, h, si.q0, row, g.do_sb, g.do_sh, g.do_sn);
    const int64_t oo = row_at(p.o_layout, b, h, si.q0, row, p.o_sb, p.o_sh, p.o_sn);
    float dsum = 0.f;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      const int col = kc * 32 + gq * 8;
      u32x4 rq = u32x4{0u, 0u, 0u, 0u}, rd = rq, ro = rq;
      if (ok) {
        rq = ld16((const char*)p.q, qo + col);
        rd = ld16((const char*)g.dout, doo + col);
        ro = ld16((const char*)p.o, oo + col);
      }
      v8 qv = __builtin_bit_cast(v8, rq);
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[e] = (T)((float)qv[e] * c);  // S in log2 units
      qf[qb][kc] = qv;
      df[qb][kc] = __builtin_bit_cast(v8, rd);
      const v8 ov = __builtin_bit_cast(v8, ro);
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum += (float)df[qb][kc][e] * (float)ov[e];
    }
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    delta[qb] = dsum;
  }

  // ---- key tiles t of [context || main], 64 keys each, K in buffer (NBUF = 2: t % 2)
  // at kbuf, V at vbuf.  issue() starts the direct loads of tile t (dma_rows); rows past
  // the segment end repeat its last row (their scores are masked to -inf, so P = 0).
  auto keys_in = [&](int t) {
    return t < nt0 ? min(kBwdBK, sc.n - t * kBwdBK) : min(kBwdBK, sm.n - (t - nt0) * kBwdBK);
  };
  auto kbuf = [&](int buf) { return smem_raw + buf * C::TILEB; };
  auto vbuf = [&](int buf) { return smem_raw + (C::DQ_NBUF + buf) * C::TILEB; };
  // the lane's direct-load offsets of a whole tile at the main segment's K row pitch (the
  // common case: every full tile whose K and V rows have that pitch)
  constexpr int NPT = PIPE ? kBwdBK / (C::RPI * kBwdNW) : 1;
  uint32_t t_off[NPT];
  const uint32_t t_rowb = __builtin_amdgcn_readfirstlane((uint32_t)sm.ksn * 2u);
  if constexpr (PIPE) dma_offsets<D, kBwdBK>(t_rowb, lane, wave, t_off);
  auto issue = [&](int t, int buf) {
    const bool m = t >= nt0;
    const int j0 = (m ? t - nt0 : t) * kBwdBK;
    if constexpr (C::PAD) {  // padded rows, one direct load per row
      const int n = m ? sm.n : sc.n;
      const char* const kp = m ? sm.k : sc.k;
      const char* const vp = m ? sm.v : sc.v;
      const int64_t ksn = m ? sm.ksn : sc.ksn, vsn = m ? sm.vsn : sc.vsn;
      const int64_t kt = m ? sm.kbase + (int64_t)j0 * ksn : key_elem(sc, sc.kbase, ksn, j0);
      const int last = min(kBwdBK, n - j0) - 1;  // rows past the segment end repeat it
      dma_rows_padded<D, kBwdBK>(uniform_ptr(kp + kt * 2), __builtin_amdgcn_readfirstlane((uint32_t)ksn * 2u), last,
                                 lds_addr(kbuf(buf)), wave, lane);
      if (!kv_same) {
        const int64_t vt = m ? sm.vbase + (int64_t)j0 * vsn : key_elem(sc, sc.vbase, vsn, j0);
        dma_rows_padded<D, kBwdBK>(uniform_ptr(vp + vt * 2), __builtin_amdgcn_readfirstlane((uint32_t)vsn * 2u), last,
                                   lds_addr(vbuf(buf)), wave, lane);
      }
    } else {
      // (segment fields picked one by one: a reference to either would put both in memory)
      const int last = min(kBwdBK, (m ? sm.n : sc.n) - j0) - 1;
      // row 0 of the tile (a paged context tile is one page): both page lookups before
      // any load is issued, so their waits wait for nothing else
      const int64_t kt = m ? sm.kbase + (int64_t)j0 * sm.ksn : key_elem(sc, sc.kbase, sc.ksn, j0);
      const int64_t vt = kv_same ? 0 : m ? sm.vbase + (int64_t)j0 * sm.vsn : key_elem(sc, sc.vbase, sc.vsn, j0);
      const char* const kp = uniform_ptr((m ? sm.k : sc.k) + kt * 2);
      const char* const vp = uniform_ptr((m ? sm.v : sc.v) + vt * 2);
      const uint32_t krowb = __builtin_amdgcn_readfirstlane((uint32_t)(m ? sm.ksn : sc.ksn) * 2u);
      const uint32_t vrowb = __builtin_amdgcn_readfirstlane((uint32_t)(m ? sm.vsn : sc.vsn) * 2u);
      if constexpr (PIPE) {
        if (last == kBwdBK - 1 && krowb == t_rowb && (kv_same || vrowb == t_rowb)) {
          dma_rows_at<D, kBwdBK>(kp, t_off, lds_addr(kbuf(buf)), wave);
          if (!kv_same) dma_rows_at<D, kBwdBK>(vp, t_off, lds_addr(vbuf(buf)), wave);
          return;
        }
      }
      dma_rows<D, kBwdBK>(kp, krowb, last, lds_addr(kbuf(buf)), wave, lane);
      if (!kv_same) dma_rows<D, kBwdBK>(vp, vrowb, last, lds_addr(vbuf(buf)), wave, lane);
    }
  };
  const TileReader<T, D> tr(l16, gq);
  auto row_frag = [&](const char* tile, int kb, int kc) { return tr.row(tile, kb, kc); };
  auto col_frag = [&](const char* tile, int ks, int db) { return tr.col(tile, ks, db); };
  // S^T = K Q^T of a tile: lane (q + 16g) reg r = S[query q][key 16kb + 4g + r]
  auto scores = [&](const char* kt, f32x4 (&s)[C::NKB][QB]) {
#pragma unroll
    for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc)
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
        const v8 a = row_frag(kt, kb, kc);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[kb][qb] = Mfma<T>::run(a, qf[qb][kc], s[kb][qb]);
      }
  };

  // ---- one pass over the key set.  With P_j = 2^(z_j - m) / l (z = scores in log2
  // units, m a running max, l = sum_j 2^(z_j - m)):
  //   dq = scale / l * sum_j 2^(z_j - m) (dP_j - delta) k_j,
  // so dq^T accumulates K^T (2^(z - m) (dP - delta))^T like the forward's O^T and is
  // rescaled with l whenever m moves (lazily: by more than kRescaleSlack).  With LSE,
  // m = lse and l = 1 throughout; in the software-pipelined tiles -lse starts the S^T
  // accumulators and -delta the dP^T ones, so the MFMAs yield z - lse and dP - delta.
  f32x4 dq[C::NDB][QB];
#pragma unroll
  for (int db = 0; db < C::NDB; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) dq[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i[QB], l_i[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = -INFINITY;
    l_i[qb] = 0.f;
    if constexpr (LSE) {  // the row's log2-sum-exp; padding rows: +inf, so P = 0
      const int row = qpos0 + (wave * QB + qb) * 16 + l16;
      m_i[qb] = row < si.len ? p.lse[(int64_t)h * p.total_q + si.q0 + row] : INFINITY;
    }
  }
  // NBUF = 2: tile t+1 loads while tile t is used; its buffer was last read by tile t-1,
  // which every wave has finished at the barrier before the issue
  if (C::DQ_NBUF == 2 && nt > 0) issue(0, 0);
  for (int t = 0; t < nt; ++t) {
    const int nk = keys_in(t);
    const int buf = C::DQ_NBUF == 2 ? (t & 1) : 0;
    if (C::DQ_NBUF == 1) {
      __syncthreads();  // the previous tile's LDS reads are done
      issue(t, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of tile t have landed
    __syncthreads();                // ... and every other wave's
    if (C::DQ_NBUF == 2 && t + 1 < nt) issue(t + 1, buf ^ 1);
    const char* const kt = kbuf(buf);
    const char* const vt = kv_same ? kt : vbuf(buf);
    if constexpr (PIPE) {
      // ---- the tile as one sequence of fenced slots (the order below is the issue
      // order): S^T slots (step kc, key block kb: kc-major, so an accumulator's next MFMA
      // is NKB slots away), then dP^T slots (key block kb, step kc: kb-major, so each
      // block's dP is done a block before the next), then dq^T slots (key step ks, column
      // block db).  The LDS read of fragment s + LEAD is issued at the top of slot s.
      // Beside the MFMAs: the tile's masked row max and lazy rescale during block 0's dP
      // (every S is done), block kb's exp / dS during block kb + 1's dP, the last block's
      // during key step 0's dq (which needs blocks 0-1 only).  No exp precedes the tile's
      // max, so a rescale never touches packed dS.
      constexpr int NSS = C::KC * C::NKB;      // S slots
      constexpr int NR = 2 * NSS;              // S slots, then dP slots
      constexpr int NS = NR + C::NKS * C::NDB;
      constexpr int LEAD = 3;
      static_assert(C::NKB == 4 && C::NKS == 2, "64-key tiles");
      f32x4 sb[C::NKB][QB], dpb[C::NKB][QB];
      u32x4 dsw[C::NKS][QB];
      v8 fr[LEAD + 1];
      auto issue = [&](int r) {
        if (r < NSS) {
          fr[r % (LEAD + 1)] = row_frag(kt, r % C::NKB, r / C::NKB);
        } else if (r < NR) {
          const int j = r - NSS;
          fr[r % (LEAD + 1)] = row_frag(vt, j / C::KC, j % C::KC);
        } else {
          const int j = r - NR;
          fr[r % (LEAD + 1)] = col_frag(kt, j / C::NDB, j % C::NDB);
        }
      };
      // the tile's row max of block qb (keys past the tile's end masked to -inf)
      auto row_max_unit = [&](int qb) {
#pragma unroll
        for (int kb = 0; kb < C::NKB; ++kb) pin(sb[kb][qb]);
        if (nk < kBwdBK) {  // a partial tile: keys past its end to -inf
          asm volatile("");  // (a real branch: full tiles skip the selects)
#pragma unroll
          for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (kb * 16 + gq * 4 + r >= nk) sb[kb][qb][r] = -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < C::NKB; ++kb)
          mx = vmax(mx, vmax(vmax(sb[kb][qb][0], sb[kb][qb][1]), vmax(sb[kb][qb][2], sb[kb][qb][3])));
        mx = lane_max_xor16_32(mx);
        pin(mx);
        return mx;
      };
      float mt[QB];
      auto rescale_unit = [&]() {
        bool grow_any = false;
        float m_new[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const bool grow = mt[qb] > m_i[qb] + kRescaleSlack;
          m_new[qb] = grow ? mt[qb] : m_i[qb];
          grow_any = grow_any || grow;
        }
        if (__builtin_amdgcn_ballot_w64(grow_any)) {
          asm volatile("");  // (a real branch: the rescale is rare)
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            const float alpha = m_i[qb] == -INFINITY ? 0.f : fast_exp2(m_i[qb] - m_new[qb]);
            m_i[qb] = m_new[qb];
            l_i[qb] *= alpha;
#pragma unroll
            for (int db = 0; db < C::NDB; ++db) dq[db][qb] *= alpha;
          }
        }
      };
      // 2^(z - m) (dP - delta) of elements r, r + 1 of key block kb, query block qb
      // (pair e: qb = e / 2, r = 2 (e % 2))
      auto soft_block = [&](int kb, int e) {
        const int qb = e >> 1, r = (e & 1) * 2;
        if (r == 0) pin(dpb[kb][qb]);
        f32x2 pv, ds;
        if constexpr (LSE) {  // the accumulators hold z - lse and dP - delta
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            pv[i] = fast_exp2(sb[kb][qb][r + i]);
            ds[i] = pv[i] * dpb[kb][qb][r + i];
          }
        } else {
          const float mref = m_i[qb] == -INFINITY ? 0.f : m_i[qb];  // no key yet: every z is -inf
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            pv[i] = fast_exp2(sb[kb][qb][r + i] - mref);
            ds[i] = pv[i] * (dpb[kb][qb][r + i] - delta[qb]);
          }
          l_i[qb] += pv[0] + pv[1];
        }
        uint32_t wd = __builtin_bit_cast(uint32_t, __builtin_convertvector(ds, typename Pair<T>::type));
        pin(wd);
        dsw[kb >> 1][qb][(kb & 1) * 2 + (r >> 1)] = wd;
      };
#pragma unroll
      for (int r = 0; r < LEAD; ++r) issue(r);
#pragma unroll
      for (int sl = 0; sl < NSS; ++sl) {
        if (sl + LEAD < NS) issue(sl + LEAD);
        const v8 a = fr[sl % (LEAD + 1)];
        const int kb = sl % C::NKB, kc = sl / C::NKB;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          sb[kb][qb] = Mfma<T>::run(a, qf[qb][kc], kc > 0 ? sb[kb][qb]
                                                   : LSE ? f32x4{-m_i[qb], -m_i[qb], -m_i[qb], -m_i[qb]}
                                                         : f32x4{0.f, 0.f, 0.f, 0.f});
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int sl = NSS; sl < NR; ++sl) {
        if (sl + LEAD < NS) issue(sl + LEAD);
        const v8 a = fr[sl % (LEAD + 1)];
        const int j = sl - NSS, kb = j / C::KC, kc = j % C::KC;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          dpb[kb][qb] = Mfma<T>::run(a, df[qb][kc], kc > 0 ? dpb[kb][qb]
                                                    : LSE ? f32x4{-delta[qb], -delta[qb], -delta[qb], -delta[qb]}
                                                          : f32x4{0.f, 0.f, 0.f, 0.f});
        if (kb == 0 && LSE) {
          // keys past a partial tile's end to -inf (P = 0), before block 0's exp
          if (j == 0 && nk < kBwdBK) {
            asm volatile("");  // (a real branch: full tiles skip the selects)
#pragma unroll
            for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
              for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  if (kb2 * 16 + gq * 4 + r >= nk) sb[kb2][qb][r] = -INFINITY;
          }
        } else if (kb == 0) {
          // the row max, then the rescale, all before block 0's exp in block 1's slots:
          // one query block per slot from slot 1 where block 0 has the slots for it,
          // else all in slot 0
          if constexpr (QB + 1 < C::KC) {
            if (j >= 1 && j <= QB) mt[j - 1] = row_max_unit(j - 1);
            if (j == QB + 1) rescale_unit();
          } else if (j == 0) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) mt[qb] = row_max_unit(qb);
            rescale_unit();
          }
        } else {  // block kb - 1's exp / dS
          const int loc = j % C::KC;
#pragma unroll
          for (int e = loc * 2 * QB / C::KC; e < (loc + 1) * 2 * QB / C::KC; ++e) soft_block(kb - 1, e);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int sl = NR; sl < NS; ++sl) {
        if (sl + LEAD < NS) issue(sl + LEAD);
        const v8 a = fr[sl % (LEAD + 1)];
        const int j = sl - NR, ks = j / C::NDB, db = j % C::NDB;
        if (ks == 0) {  // the last block's exp / dS
#pragma unroll
          for (int e = j * 2 * QB / C::NDB; e < (j + 1) * 2 * QB / C::NDB; ++e) soft_block(C::NKB - 1, e);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) dq[db][qb] = Mfma<T>::run(a, __builtin_bit_cast(v8, dsw[ks][qb]), dq[db][qb]);
        __builtin_amdgcn_sched_barrier(0);
      }
      continue;
    }
    f32x4 s[C::NKB][QB], dp[C::NKB][QB];
    scores(kt, s);
    // dP^T = V dO^T, same layout as S^T
#pragma unroll
    for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) dp[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc)
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
        const v8 a = row_frag(vt, kb, kc);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) dp[kb][qb] = Mfma<T>::run(a, df[qb][kc], dp[kb][qb]);
      }
    if constexpr (LSE) {
      if (nk < kBwdBK) {  // a partial tile: keys past its end to -inf (P = 0)
        asm volatile("");  // (a real branch: full tiles skip the selects)
#pragma unroll
        for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (kb * 16 + gq * 4 + r >= nk) s[kb][qb][r] = -INFINITY;
      }
    } else {
    // running max (row-uniform after the xor steps) and lazy rescale
    bool grow_any = false;
    float m_new[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float z = kb * 16 + gq * 4 + r < nk ? s[kb][qb][r] : -INFINITY;
          s[kb][qb][r] = z;
          mx = fmaxf(mx, z);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const bool grow = mx > m_i[qb] + kRescaleSlack;
      m_new[qb] = grow ? mx : m_i[qb];
      grow_any = grow_any || grow;
    }
    if (__builtin_amdgcn_ballot_w64(grow_any)) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const float alpha = m_i[qb] == -INFINITY ? 0.f : fast_exp2(m_i[qb] - m_new[qb]);
        m_i[qb] = m_new[qb];
        l_i[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) dq[db][qb] *= alpha;
      }
    }
    }
    // 2^(z - m) (dP - delta), packed as B operands: element 4h + r of step ks is key
    // 32ks + 16h + 4g + r
    v8 dsf[C::NKS][QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      // no key yet: every z is -inf (LSE: m is the row's statistic, +inf for padding rows)
      const float mref = !LSE && m_i[qb] == -INFINITY ? 0.f : m_i[qb];
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = fast_exp2(s[kb][qb][r] - mref);
          rs += pv;
          dsf[kb >> 1][qb][(kb & 1) * 4 + r] = (T)(pv * (dp[kb][qb][r] - delta[qb]));
        }
      if (!LSE) l_i[qb] += rs;
    }
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks)
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        const v8 a = col_frag(kt, ks, db);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) dq[db][qb] = Mfma<T>::run(a, dsf[ks][qb], dq[db][qb]);
      }
  }
  // row statistics for the dK / dV kernel: lse = m + log2(l) (no keys: +inf, P = 0)
  float* const st_lse = (float*)g.workspace;
  float* const st_delta = st_lse + (int64_t)p.H * p.total_q;
  float dq_mul[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    float l = l_i[qb];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const bool any = l > 0.f;
    dq_mul[qb] = LSE ? p.scale : any ? p.scale / l : 0.f;
    const int row = qpos0 + (wave * QB + qb) * 16 + l16;
    if (gq == 0 && row < si.len) {
      const int64_t at = (int64_t)h * p.total_q + si.q0 + row;
      if (!LSE) st_lse[at] = any ? m_i[qb] + __log2f(l) : INFINITY;
      // the dK / dV kernel's dS = P (scale dP - scale delta); the latent's kernel (whose
      // spills move with any change of its code) keeps delta and multiplies by scale
      st_delta[at] = C::MLA_ONLY ? delta[qb] : delta[qb] * p.scale;
    }
  }

  // ---- dq rows: lane (q + 16g) holds dq[q][16db + 4g .. +4]
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = qpos0 + (wave * QB + qb) * 16 + l16;
    if (row >= si.len) continue;
    const int64_t off = row_at(p.q_layout, b, h, si.q0, row, g.dq_sb, g.dq_sh, g.dq_sn);
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      T v4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = (T)(dq[db][qb][r] * dq_mul[qb]);
      *(u32x2*)((char*)g.dq + (off + db * 16 + gq * 4) * 2) = *(const u32x2*)v4;
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV kernel, context keys and main keys in one grid (units, key heads): the first
// units are key tiles of the context batches (unit table), the following ones key tiles
// of the main keys (per sequence from the unit table, or with CAUSAL the tiles of the
// causal token range).  Context tiles go first: a shared context's tiles take the
// queries of every sequence and are the longest units.
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(kBwdNW * 64, BwdCfg<D>::WPS) void attn_bwd_dkv_kernel(const fmlm_attn_params p,
                                                                      const fmlm_attn_grads g, int n_ctx,
                                                                      const int32_t* krec, int nk) {
  typedef BwdCfg<D> C;
  typedef typename Mfma<T>::v8 v8;
  extern __shared__ __align__(16) char smem_raw[];
  // step buffer i: QS rows of Q, QS rows of dO (pitch ROWB), then QS lse and QS delta
  auto qbuf = [&](int i) { return smem_raw + i * C::DKV_SB; };
  auto obuf = [&](int i) { return smem_raw + i * C::DKV_SB + C::STEPB; };
  auto lse_s = [&](int i) { return (float*)(smem_raw + i * C::DKV_SB + 2 * C::STEPB); };
  auto dl_s = [&](int i) { return lse_s(i) + C::QS; };

  const bool mla = C::MLA_ONLY || (p.flags & FMLM_FLAG_MLA);
  // software-pipelined step (below) for 64-row steps of unpadded tiles
  constexpr bool PIPE = !C::PAD && !C::MLA_ONLY && C::QS == 64;
  KeyUnit ku;
  if (!resolve_key_unit<CAUSAL>(p, g, n_ctx, krec, nk, ku)) return;
  const BSeg& s = ku.s;
  const int j0 = ku.j0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, gq = lane >> 4;
  const float c = p.scale * kLog2e;
  // the row statistics: the forward's log2-sum-exp when it stored them, else the dq
  // kernel's; delta from the dq kernel
  const float* const st_delta = (const float*)g.workspace + (int64_t)p.H * p.total_q;
  const float* const st_lse = p.lse ? (const float*)p.lse : (const float*)g.workspace;

  // this lane's keys (B-operand / accumulator column of each of the wave's KB 16-key
  // blocks) and their K, V fragments: kf[kb][kc] = K[key][kc*32 + 8g .. +8]
  constexpr int KB = C::KB;
  int key[KB];
  bool kok[KB];
  v8 kf[KB][C::KC], vf[KB][C::KC];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    key[kb] = j0 + (wave * KB + kb) * 16 + l16;
    kok[kb] = key[kb] < s.n;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      u32x4 rk = u32x4{0u, 0u, 0u, 0u}, rv = rk;
      if (kok[kb]) {
        rk = ld16(s.k, key_elem(s, s.kbase, s.ksn, key[kb]) + kc * 32 + gq * 8);
        if (!mla) rv = ld16(s.v, key_elem(s, s.vbase, s.vsn, key[kb]) + kc * 32 + gq * 8);
      }
      kf[kb][kc] = __builtin_bit_cast(v8, rk);
      vf[kb][kc] = mla ? kf[kb][kc] : __builtin_bit_cast(v8, rv);
    }
  }
  f32x4 dkt[KB][C::NDB], dvt[KB][C::MLA_ONLY ? 1 : C::NDB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      dkt[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (!C::MLA_ONLY) dvt[kb][db] = dkt[kb][db];
    }

  // Query steps: (head hq, sequence b, rows [p0, p0 + QS)) over every sequence whose
  // queries attend to these keys, heads outermost.  prep() starts the loads of a step:
  // its rows by direct loads into step buffer buf (rows past the sequence end repeat its
  // last row; their lse is +inf, so P = dS = 0) and its lse / delta into registers, which
  // go to LDS at the top of the step's iteration.  The latent (PAD) stages everything
  // through registers into its single buffer after the previous step's reads.
  const int hq_lo = ku.shared ? 0 : ku.kh, hq_hi = ku.shared ? p.H : ku.kh + 1;
  const QuerySteps steps{&p, &ku, hq_hi, C::QS};
  // the lane's direct-load offsets of a whole step of Q and of dO rows
  constexpr int NPQ = PIPE ? C::QS / (C::RPI * kBwdNW) : 1;
  uint32_t q_off[NPQ], o_off[NPQ];
  if constexpr (PIPE) {
    dma_offsets<D, C::QS>(__builtin_amdgcn_readfirstlane((uint32_t)p.q_sn * 2u), lane, wave, q_off);
    dma_offsets<D, C::QS>(__builtin_amdgcn_readfirstlane((uint32_t)g.do_sn * 2u), lane, wave, o_off);
  }
  float lreg = INFINITY, dlreg = 0.f;
  // si: the ranges of st's sequence
  auto prep = [&](const QStep& st, const SeqInfo& si, int buf) {
    if (tid < C::QS) {
      const int pos = st.p0 + tid;
      const bool ok = pos < si.len;
      const int64_t at = (int64_t)st.hq * p.total_q + si.q0 + pos;
      lreg = ok ? st_lse[at] : INFINITY;  // padding rows: P = 0
      dlreg = ok ? st_delta[at] : 0.f;
    }
    if constexpr (C::PAD) {  // padded rows, one direct load per row
      const int last = min(C::QS, si.len - st.p0) - 1;
      const int64_t qe = row_at(p.q_layout, st.b, st.hq, si.q0, st.p0, p.q_sb, p.q_sh, p.q_sn);
      const int64_t de = row_at(p.o_layout, st.b, st.hq, si.q0, st.p0, g.do_sb, g.do_sh, g.do_sn);
      dma_rows_padded<D, C::QS>(uniform_ptr((const char*)p.q + qe * 2), __builtin_amdgcn_readfirstlane((uint32_t)p.q_sn * 2u),
                                last, lds_addr(qbuf(buf)), wave, lane);
      dma_rows_padded<D, C::QS>(uniform_ptr((const char*)g.dout + de * 2),
                                __builtin_amdgcn_readfirstlane((uint32_t)g.do_sn * 2u), last, lds_addr(obuf(buf)), wave,
                                lane);
    } else {
      const int last = min(C::QS, si.len - st.p0) - 1;
      const int64_t qe = row_at(p.q_layout, st.b, st.hq, si.q0, st.p0, p.q_sb, p.q_sh, p.q_sn);
      const int64_t de = row_at(p.o_layout, st.b, st.hq, si.q0, st.p0, g.do_sb, g.do_sh, g.do_sn);
      const char* const qs = uniform_ptr((const char*)p.q + qe * 2);
      const char* const ds = uniform_ptr((const char*)g.dout + de * 2);
      if constexpr (PIPE) {
        if (last == C::QS - 1) {  // a whole step: the precomputed offsets
          dma_rows_at<D, C::QS>(qs, q_off, lds_addr(qbuf(buf)), wave);
          dma_rows_at<D, C::QS>(ds, o_off, lds_addr(obuf(buf)), wave);
          return;
        }
      }
      dma_rows<D, C::QS>(qs, __builtin_amdgcn_readfirstlane((uint32_t)p.q_sn * 2u), last, lds_addr(qbuf(buf)), wave, lane);
      dma_rows<D, C::QS>(ds, __builtin_amdgcn_readfirstlane((uint32_t)g.do_sn * 2u), last, lds_addr(obuf(buf)), wave, lane);
    }
  };
  // Pipelined kernels: a step's row 0 in Q, dO and the row statistics, derived once per
  // (head, sequence) and then advanced by one step per step; prep_rows() is prep() with
  // them (the other kernels compute them per step: they have no scalar registers to spare)
  struct StepRows {
    const char* q;
    const char* d;
    int64_t at;  // index of the row statistics
  };
  auto step_rows = [&](const QStep& st, const SeqInfo& si) {
    StepRows r;
    r.q = uniform_ptr((const char*)p.q + row_at(p.q_layout, st.b, st.hq, si.q0, st.p0, p.q_sb, p.q_sh, p.q_sn) * 2);
    r.d = uniform_ptr((const char*)g.dout + row_at(p.o_layout, st.b, st.hq, si.q0, st.p0, g.do_sb, g.do_sh, g.do_sn) * 2);
    r.at = (int64_t)st.hq * p.total_q + si.q0 + st.p0;
    return r;
  };
  auto next_rows = [&](const StepRows& r) {
    return StepRows{uniform_ptr(r.q + (int64_t)C::QS * p.q_sn * 2), uniform_ptr(r.d + (int64_t)C::QS * g.do_sn * 2),
                    r.at + C::QS};
  };
  auto prep_rows = [&](const QStep& st, const SeqInfo& si, const StepRows& rows, int buf) {
    if constexpr (PIPE) {
      if (tid < C::QS) {
        const bool ok = st.p0 + tid < si.len;
        lreg = ok ? st_lse[rows.at + tid] : INFINITY;  // padding rows: P = 0
        dlreg = ok ? st_delta[rows.at + tid] : 0.f;
      }
      const int last = min(C::QS, si.len - st.p0) - 1;
      if (last == C::QS - 1) {  // a whole step: the precomputed offsets
        dma_rows_at<D, C::QS>(rows.q, q_off, lds_addr(qbuf(buf)), wave);
        dma_rows_at<D, C::QS>(rows.d, o_off, lds_addr(obuf(buf)), wave);
        return;
      }
      dma_rows<D, C::QS>(rows.q, __builtin_amdgcn_readfirstlane((uint32_t)p.q_sn * 2u), last, lds_addr(qbuf(buf)), wave, lane);
      dma_rows<D, C::QS>(rows.d, __builtin_amdgcn_readfirstlane((uint32_t)g.do_sn * 2u), last, lds_addr(obuf(buf)), wave, lane);
    }
  };

  const TileReader<T, D> tr(l16, gq);

  // the ranges of the current and the next step's sequences are read once per sequence:
  // consecutive steps of one sequence reuse them
  // the first step: sequence b_lo of the first head, with its ranges from the unit record
  QStep cur{ku.b_lo < ku.b_hi ? hq_lo : hq_hi, ku.b_lo, 0};
  SeqInfo si_cur = ku.si_lo;
  StepRows rows_cur{};
  int buf = 0;
  if constexpr (PIPE) {
    if (cur.hq < hq_hi) {
      rows_cur = step_rows(cur, si_cur);
      prep_rows(cur, si_cur, rows_cur, 0);
    }
  } else {
    if (cur.hq < hq_hi) prep(cur, si_cur, 0);
  }
  while (cur.hq < hq_hi) {
    const QStep nxt = steps.next(cur, si_cur.len);
    const SeqInfo si_nxt = (nxt.hq < hq_hi && nxt.b != cur.b) ? seq_info(p, nxt.b) : si_cur;
    StepRows rows_nxt{};
    if constexpr (PIPE) {
      if (nxt.b == cur.b && nxt.hq == cur.hq)
        rows_nxt = next_rows(rows_cur);
      else if (nxt.hq < hq_hi)
        rows_nxt = step_rows(nxt, si_nxt);
    }
    const int lim = ku.causal_main ? si_cur.mainlen : 0x7fffffff;
    if (tid < C::QS) {  // this buffer's statistics were last read two steps ago
      lse_s(buf)[tid] = lreg;
      dl_s(buf)[tid] = dlreg;
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the step have landed
    __syncthreads();                // ... and every other wave's
    // the other buffer was last read by the previous step, which every wave has finished
    if constexpr (PIPE) {
      if (nxt.hq < hq_hi) prep_rows(nxt, si_nxt, rows_nxt, buf ^ 1);
    } else {
      if (nxt.hq < hq_hi) prep(nxt, si_nxt, buf ^ 1);
    }
    const char* const qt = qbuf(buf);
    const char* const ot = obuf(buf);
    const float* const ls = lse_s(buf);
    const float* const dls = dl_s(buf);

    if constexpr (PIPE) {
      // ---- the step as one sequence of slots fenced by sched_barrier (the order below is
      // the issue order).  Slot s runs the KB MFMAs of operand fragment s: row slots
      // (row block rb of 16 query rows, step kc, Q -> S^T or dO -> dP^T; lane (key + 16g)
      // reg r = row 16rb + 4g + r), then column slots (32-row group grp, column block db,
      // dO^T -> dV^T with P or Q^T -> dK^T with dS).  The LDS read of fragment s + LEAD is
      // issued at the top of slot s.  The softmax of row block rb (P and dS, packed as B
      // operands: element 4h + r of group rb / 2, h = rb % 2) runs beside the MFMAs of
      // the next row block, the last block's beside the first group's column slots, so
      // every column slot finds its operands done.
      constexpr int NRB = C::QS / 16;
      constexpr int RBS = 2 * C::KC;      // slots per row block
      constexpr int NR = NRB * RBS;       // row slots
      constexpr int NCS = 2 * C::NDB;     // column slots per group
      constexpr int NS = NR + 2 * NCS;
      constexpr int LEAD = 3;
      constexpr int NE2 = KB * 2;         // softmax element pairs per row block and lane
      f32x4 sc[NRB][KB], dp[NRB][KB], L4[NRB], D4[NRB];
      u32x4 pbw[2][KB], dsw[2][KB];
      v8 fr[LEAD + 1];
      // keys this step does not see (past the segment, or causal: not before cu[b+1]) start
      // their S^T accumulators at an infinity that the scale turns into -inf, so their P
      // is 0 without a select per element (a zero scale is replaced by a tiny one, which
      // leaves every finite score's 2^(s c) at 1 in fp32)
      const float cm = c != 0.f ? c : 1e-30f;
      f32x4 kin4[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const float kin = (kok[kb] && key[kb] < lim) ? 0.f : cm > 0.f ? -INFINITY : INFINITY;
        kin4[kb] = f32x4{kin, kin, kin, kin};
      }
      auto issue = [&](int r) {
        if (r < NR) {
          const int rb = r / RBS, kc = (r % RBS) >> 1;
          fr[r % (LEAD + 1)] = tr.row((r & 1) ? ot : qt, rb, kc);
        } else {
          const int j = r - NR, grp = j / NCS, db = (j % NCS) >> 1;
          fr[r % (LEAD + 1)] = tr.col((j & 1) ? qt : ot, grp, db);
        }
      };
      // P and dS of elements r, r + 1 of key block kb (pair e2 = 2 kb + r / 2) of row block rb
      auto soft_pair = [&](int rb, int e2) {
        const int kb = e2 >> 1, r = (e2 & 1) * 2, grp = rb >> 1, hh = rb & 1;
        if (r == 0) {
          pin(sc[rb][kb]);
          pin(dp[rb][kb]);
        }
        f32x2 pv, ds;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          pv[i] = fast_exp2(fmaf(sc[rb][kb][r + i], cm, -L4[rb][r + i]));  // masked keys: 2^-inf = 0
          ds[i] = pv[i] * fmaf(dp[rb][kb][r + i], p.scale, -D4[rb][r + i]);
        }
        uint32_t wp = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv, typename Pair<T>::type));
        uint32_t wd = __builtin_bit_cast(uint32_t, __builtin_convertvector(ds, typename Pair<T>::type));
        pin(wp);
        pin(wd);
        pbw[grp][kb][hh * 2 + (r >> 1)] = wp;
        dsw[grp][kb][hh * 2 + (r >> 1)] = wd;
      };
#pragma unroll
      for (int r = 0; r < LEAD; ++r) issue(r);
      // two loops (row slots, column slots): one loop over all of them is too large to
      // unroll, and the fragment ring must stay in registers
#pragma unroll
      for (int sl = 0; sl < NR; ++sl) {
        if (sl + LEAD < NS) issue(sl + LEAD);
        const v8 a = fr[sl % (LEAD + 1)];
        {
          const int rb = sl / RBS, kc = (sl % RBS) >> 1;
          if (rb > 0 && sl % RBS == 0) {  // statistics of the block whose softmax runs here
            L4[rb - 1] = *(const f32x4*)(ls + (rb - 1) * 16 + gq * 4);
            D4[rb - 1] = *(const f32x4*)(dls + (rb - 1) * 16 + gq * 4);
          }
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            if ((sl & 1) == 0)
              sc[rb][kb] = Mfma<T>::run(a, kf[kb][kc], kc == 0 ? kin4[kb] : sc[rb][kb]);
            else
              dp[rb][kb] = Mfma<T>::run(a, vf[kb][kc], kc == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : dp[rb][kb]);
          }
          if (rb > 0) {
            const int loc = sl % RBS;
#pragma unroll
            for (int e2 = loc * NE2 / RBS; e2 < (loc + 1) * NE2 / RBS; ++e2) soft_pair(rb - 1, e2);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int sl = NR; sl < NS; ++sl) {
        if (sl + LEAD < NS) issue(sl + LEAD);
        const v8 a = fr[sl % (LEAD + 1)];
        {
          const int j = sl - NR, grp = j / NCS, db = (j % NCS) >> 1;
          if (j == 0) {
            L4[NRB - 1] = *(const f32x4*)(ls + (NRB - 1) * 16 + gq * 4);
            D4[NRB - 1] = *(const f32x4*)(dls + (NRB - 1) * 16 + gq * 4);
          }
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            if ((j & 1) == 0) {  // (MLA: dV^T joins dK^T after the last step)
              dvt[kb][db] = Mfma<T>::run(a, __builtin_bit_cast(v8, pbw[grp][kb]), dvt[kb][db]);
            } else {
              dkt[kb][db] = Mfma<T>::run(a, __builtin_bit_cast(v8, dsw[grp][kb]), dkt[kb][db]);
            }
          }
          if (grp == 0) {
#pragma unroll
            for (int e2 = j * NE2 / NCS; e2 < (j + 1) * NE2 / NCS; ++e2) soft_pair(NRB - 1, e2);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
    // per 32-row group: S and dP for its two 16-row halves (lane (key + 16g) reg r = row
    // 32grp + 16h + 4g + r), P and dS packed as B operands (element 4h + r), then the
    // dV / dK products.  Each fragment read from LDS feeds the KB key blocks.
#pragma unroll
    for (int grp = 0; grp < C::QS / 32; ++grp) {
    v8 pb[KB], dsb[KB];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      f32x4 sc[KB], dp[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[kb] = sc[kb];
      }
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc) {
        const v8 aq = tr.row(qt, grp * 2 + hh, kc);
        const v8 ao = tr.row(ot, grp * 2 + hh, kc);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          sc[kb] = Mfma<T>::run(aq, kf[kb][kc], sc[kb]);
          dp[kb] = Mfma<T>::run(ao, vf[kb][kc], dp[kb]);
        }
      }
      const f32x4 L4 = *(const f32x4*)(ls + grp * 32 + hh * 16 + gq * 4);
      const f32x4 D4 = *(const f32x4*)(dls + grp * 32 + hh * 16 + gq * 4);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const bool kvalid = kok[kb] && key[kb] < lim;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = kvalid ? fast_exp2(fmaf(sc[kb][r], c, -L4[r])) : 0.f;
          pb[kb][hh * 4 + r] = (T)pv;
          if constexpr (C::MLA_ONLY)
            dsb[kb][hh * 4 + r] = (T)(pv * (dp[kb][r] - D4[r]) * p.scale);
          else
            dsb[kb][hh * 4 + r] = (T)(pv * fmaf(dp[kb][r], p.scale, -D4[r]));
        }
      }
    }
    // dV^T += dO^T P and dK^T += Q^T dS (MLA: both into dK)
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      const v8 ao = tr.col(ot, grp, db);
      const v8 aq = tr.col(qt, grp, db);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (mla) {
          dkt[kb][db] = Mfma<T>::run(ao, pb[kb], dkt[kb][db]);
        } else if constexpr (!C::MLA_ONLY) {
          dvt[kb][db] = Mfma<T>::run(ao, pb[kb], dvt[kb][db]);
        }
        dkt[kb][db] = Mfma<T>::run(aq, dsb[kb], dkt[kb][db]);
      }
    }
    }
    }
    buf ^= 1;
    cur = nxt;
    si_cur = si_nxt;
    if constexpr (PIPE) rows_cur = rows_nxt;
  }

  if constexpr (PIPE) {  // the pipelined steps keep dO^T P apart; with V = K it is part of dK
    if (mla)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) dkt[kb][db] += dvt[kb][db];
  }

  // ---- rows: lane (key + 16g) holds d?[key][16db + 4g .. +4].  The paged / contiguous
  // choice sits outside the block loops, so each loop converts and stores one 16-column
  // block at a time (with the branch inside, the 512-wide latent read every accumulator
  // out at once and spilled).  At D >= 256 the keys are laundered, so that their
  // addresses are recomputed here rather than kept live across the step loop from the K
  // loads, which spilled them (at D <= 128 the registers this frees changed the step
  // loop's allocation: the D = 64 kernel went to four waves per SIMD and ran slower)
  int kst[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    kst[kb] = key[kb];
    if constexpr (D >= 256) asm volatile("" : "+v"(kst[kb]));
  }
  if (s.pages) {  // float32 gradients, added atomically
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (!kok[kb]) continue;
      float* const dkf = (float*)s.dk + key_elem(s, s.dkbase, s.dksn, kst[kb]) + gq * 4;
      float* const dvf = (float*)s.dv + key_elem(s, s.dvbase, s.dvsn, kst[kb]) + gq * 4;
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
#pragma unroll
        for (int r = 0; r < 4; ++r) atomicAdd(dkf + db * 16 + r, dkt[kb][db][r]);
        if constexpr (!C::MLA_ONLY) {
          if (!mla)
#pragma unroll
            for (int r = 0; r < 4; ++r) atomicAdd(dvf + db * 16 + r, dvt[kb][db][r]);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    if (!kok[kb]) continue;
    char* const dkr = s.dk + (s.dkbase + (int64_t)kst[kb] * s.dksn + gq * 4) * 2;
    char* const dvr = s.dv + (s.dvbase + (int64_t)kst[kb] * s.dvsn + gq * 4) * 2;
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      T k4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = dkt[kb][db][r];
        // the latent's accumulators fill the AGPRs: read each one out where it is stored
        // (copied out all at once after the step loop, they did not fit the VGPRs)
        if constexpr (C::MLA_ONLY) asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(dkt[kb][db][r]));
        k4[r] = (T)x;
      }
      *(u32x2*)(dkr + db * 32) = *(const u32x2*)k4;
      if constexpr (!C::MLA_ONLY) {
        if (!mla) {
          T v4[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v4[r] = (T)dvt[kb][db][r];
          *(u32x2*)(dvr + db * 32) = *(const u32x2*)v4;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// SIMT backward (fp32 inputs, and head dims without an MFMA kernel): the same two-kernel
// split as above.  TPR threads per query row (dq) or per key row (dK / dV), each holding
// DPT dims; a row's partial dot products meet through xor shuffles inside its TPR lanes,
// and the staged tiles are fp32 in LDS, read as float4.
// ---------------------------------------------------------------------------
template <int D>
struct SimtBwdCfg {
  static constexpr int TPR = D / 4 < 16 ? D / 4 : 16;
  static constexpr int DPT = D / TPR;
  static constexpr int NT = 256;
  static constexpr int R = NT / TPR;                       // query rows / keys per workgroup
  static constexpr int BKS = 4096 / D < 64 ? 4096 / D : 64;  // query rows per dkv step
  static constexpr int DQK = BKS < 32 ? BKS : 32;            // keys per dq tile (scores in registers)
  static constexpr int DQ_LDS = 2 * DQK * D * 4;
  static constexpr int DKV_LDS = 2 * BKS * D * 4 + 2 * BKS * 4;
  static_assert(DPT % 4 == 0 && (TPR & (TPR - 1)) == 0, "simt tiling");
};

template <typename T>
FMLM_DEV float4 ld4f(const T* p) {
  return float4{(float)p[0], (float)p[1], (float)p[2], (float)p[3]};
}
template <>
FMLM_DEV float4 ld4f<float>(const float* p) {
  return *(const float4*)p;
}

// sum over the TPR lanes of a row
template <int TPR>
FMLM_DEV float row_sum(float x) {
#pragma unroll
  for (int off = 1; off < TPR; off <<= 1) x += __shfl_xor(x, off);
  return x;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_simt_kernel(const fmlm_attn_params p, const fmlm_attn_grads g,
                                                               const int32_t* qrec, int nq) {
  typedef SimtBwdCfg<D> C;
  extern __shared__ __align__(16) char smem_raw[];
  float* const Kf = (float*)smem_raw;
  float* const Vf = Kf + C::DQK * D;

  int u, h;
  grid_unit((unsigned)p.H, u, h);
  if (u >= nq) return;
  int rec[9];  // the unit's record (query_record)
  load_record(qrec + (int64_t)u * kRecInts, rec);
  const int b = rec[0];
  if (b < 0) return;
  const int qpos0 = rec[1];
  const SeqInfo si = rec_seq_info(rec + 2);
  const int tid = threadIdx.x, row = tid / C::TPR, d0 = (tid % C::TPR) * C::DPT;
  const int pos = qpos0 + row;
  const bool ok = pos < si.len;
  const float c = p.scale * kLog2e;
  const bool kv_same = p.flags & FMLM_FLAG_MLA;

  float q[C::DPT], dof[C::DPT], acc[C::DPT];
  float dsum = 0.f;
  {
    const T* qp = (const T*)p.q + row_at(p.q_layout, b, h, si.q0, pos, p.q_sb, p.q_sh, p.q_sn) + d0;
    const T* dp = (const T*)g.dout + row_at(p.o_layout, b, h, si.q0, pos, g.do_sb, g.do_sh, g.do_sn) + d0;
    const T* op = (const T*)p.o + row_at(p.o_layout, b, h, si.q0, pos, p.o_sb, p.o_sh, p.o_sn) + d0;
#pragma unroll
    for (int d = 0; d < C::DPT; d += 4) {
      const float4 z4 = float4{0.f, 0.f, 0.f, 0.f};
      const float4 a = ok ? ld4f(qp + d) : z4, e = ok ? ld4f(dp + d) : z4, o = ok ? ld4f(op + d) : z4;
      q[d] = a.x, q[d + 1] = a.y, q[d + 2] = a.z, q[d + 3] = a.w;
      dof[d] = e.x, dof[d + 1] = e.y, dof[d + 2] = e.z, dof[d + 3] = e.w;
      dsum += e.x * o.x + e.y * o.y + e.z * o.z + e.w * o.w;
      acc[d] = acc[d + 1] = acc[d + 2] = acc[d + 3] = 0.f;
    }
  }
  const float delta = row_sum<C::TPR>(dsum);

  const BSeg sc = ctx_seg_at(p, g, rec[6], h, rec[7], rec[8]);
  const BSeg sm = main_seg_at(p, g, b, h, si);
  const int nt0 = (sc.n + C::DQK - 1) / C::DQK;
  const int nt = nt0 + (sm.n + C::DQK - 1) / C::DQK;
  float m_i = -INFINITY, l_i = 0.f;
  for (int t = 0; t < nt; ++t) {
    const bool m = t >= nt0;
    const int j0 = (m ? t - nt0 : t) * C::DQK, n = m ? sm.n : sc.n;
    const int nk = min(C::DQK, n - j0);
    __syncthreads();
    for (int e = tid * 4; e < C::DQK * D; e += C::NT * 4) {
      const int kk = e / D, d = e % D, key = j0 + kk;
      float4 kv = float4{0.f, 0.f, 0.f, 0.f}, vv = kv;
      if (kk < nk) {
        kv = m ? ld4f((const T*)sm.k + sm.kbase + (int64_t)key * sm.ksn + d)
               : ld4f((const T*)sc.k + key_elem(sc, sc.kbase, sc.ksn, key) + d);
        vv = kv_same ? kv
             : m     ? ld4f((const T*)sm.v + sm.vbase + (int64_t)key * sm.vsn + d)
                     : ld4f((const T*)sc.v + key_elem(sc, sc.vbase, sc.vsn, key) + d);
      }
      *(float4*)(Kf + e) = kv;
      *(float4*)(Vf + e) = vv;
    }
    __syncthreads();
    float z[C::DQK], dpv[C::DQK];
    float mx = -INFINITY;
#pragma unroll
    for (int kk = 0; kk < C::DQK; ++kk) {
      float sdot = 0.f, pdot = 0.f;
#pragma unroll
      for (int d = 0; d < C::DPT; d += 4) {
        const float4 k4 = *(const float4*)(Kf + kk * D + d0 + d);
        const float4 v4 = *(const float4*)(Vf + kk * D + d0 + d);
        sdot += q[d] * k4.x + q[d + 1] * k4.y + q[d + 2] * k4.z + q[d + 3] * k4.w;
        pdot += dof[d] * v4.x + dof[d + 1] * v4.y + dof[d + 2] * v4.z + dof[d + 3] * v4.w;
      }
      sdot = row_sum<C::TPR>(sdot);
      dpv[kk] = row_sum<C::TPR>(pdot);
      z[kk] = kk < nk ? sdot * c : -INFINITY;
      mx = fmaxf(mx, z[kk]);
    }
    const float m_new = fmaxf(m_i, mx);
    const float alpha = m_i == -INFINITY ? 0.f : fast_exp2(m_i - m_new);
    const float mref = m_new == -INFINITY ? 0.f : m_new;
    l_i *= alpha;
#pragma unroll
    for (int d = 0; d < C::DPT; ++d) acc[d] *= alpha;
    m_i = m_new;
#pragma unroll
    for (int kk = 0; kk < C::DQK; ++kk) {
      const float pv = fast_exp2(z[kk] - mref);
      l_i += pv;
      const float gq = pv * (dpv[kk] - delta);
#pragma unroll
      for (int d = 0; d < C::DPT; d += 4) {
        const float4 k4 = *(const float4*)(Kf + kk * D + d0 + d);
        acc[d] += gq * k4.x;
        acc[d + 1] += gq * k4.y;
        acc[d + 2] += gq * k4.z;
        acc[d + 3] += gq * k4.w;
      }
    }
  }
  if (!ok) return;
  if (d0 == 0) {
    float* const st_lse = (float*)g.workspace;
    const int64_t at = (int64_t)h * p.total_q + si.q0 + pos;
    st_lse[at] = l_i > 0.f ? m_i + __log2f(l_i) : INFINITY;
    st_lse[(int64_t)p.H * p.total_q + at] = delta;
  }
  const float mul = l_i > 0.f ? p.scale / l_i : 0.f;
  T* dqp = (T*)g.dq + row_at(p.q_layout, b, h, si.q0, pos, g.dq_sb, g.dq_sh, g.dq_sn) + d0;
#pragma unroll
  for (int d = 0; d < C::DPT; ++d) dqp[d] = (T)(acc[d] * mul);
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dkv_simt_kernel(const fmlm_attn_params p, const fmlm_attn_grads g,
                                                                int n_ctx, const int32_t* krec, int nk) {
  typedef SimtBwdCfg<D> C;
  constexpr int QS = C::BKS;
  extern __shared__ __align__(16) char smem_raw[];
  float* const Qf = (float*)smem_raw;
  float* const Of = Qf + QS * D;
  float* const lse_s = Of + QS * D;
  float* const dl_s = lse_s + QS;

  const bool mla = p.flags & FMLM_FLAG_MLA;
  KeyUnit ku;
  if (!resolve_key_unit<CAUSAL>(p, g, n_ctx, krec, nk, ku)) return;
  const BSeg& s = ku.s;
  const int tid = threadIdx.x, d0 = (tid % C::TPR) * C::DPT;
  const int key = ku.j0 + tid / C::TPR;
  const bool kok = key < s.n;
  const float c = p.scale * kLog2e;
  // the row statistics: the forward's log2-sum-exp when it stored them, else the dq
  // kernel's; delta from the dq kernel
  const float* const st_delta = (const float*)g.workspace + (int64_t)p.H * p.total_q;
  const float* const st_lse = p.lse ? (const float*)p.lse : (const float*)g.workspace;

  float kf[C::DPT], vf[C::DPT], dk[C::DPT], dv[C::DPT];
#pragma unroll
  for (int d = 0; d < C::DPT; d += 4) {
    const float4 z4 = float4{0.f, 0.f, 0.f, 0.f};
    const float4 a = kok ? ld4f((const T*)s.k + key_elem(s, s.kbase, s.ksn, key) + d0 + d) : z4;
    const float4 e = kok && !mla ? ld4f((const T*)s.v + key_elem(s, s.vbase, s.vsn, key) + d0 + d) : a;
    kf[d] = a.x, kf[d + 1] = a.y, kf[d + 2] = a.z, kf[d + 3] = a.w;
    vf[d] = e.x, vf[d + 1] = e.y, vf[d + 2] = e.z, vf[d + 3] = e.w;
    dk[d] = dk[d + 1] = dk[d + 2] = dk[d + 3] = 0.f;
    dv[d] = dv[d + 1] = dv[d + 2] = dv[d + 3] = 0.f;
  }

  const int hq_lo = ku.shared ? 0 : ku.kh, hq_hi = ku.shared ? p.H : ku.kh + 1;
  const QuerySteps steps{&p, &ku, hq_hi, QS};
  for (QStep cur = steps.first_from(hq_lo, ku.b_lo); cur.hq < hq_hi; cur = steps.next(cur)) {
    const SeqInfo si = seq_info(p, cur.b);
    __syncthreads();  // the previous step's LDS reads are done
    for (int e = tid * 4; e < QS * D; e += C::NT * 4) {
      const int r = e / D, d = e % D, pos = cur.p0 + r;
      float4 a = float4{0.f, 0.f, 0.f, 0.f}, o = a;
      if (pos < si.len) {
        a = ld4f((const T*)p.q + row_at(p.q_layout, cur.b, cur.hq, si.q0, pos, p.q_sb, p.q_sh, p.q_sn) + d);
        o = ld4f((const T*)g.dout + row_at(p.o_layout, cur.b, cur.hq, si.q0, pos, g.do_sb, g.do_sh, g.do_sn) + d);
      }
      *(float4*)(Qf + e) = a;
      *(float4*)(Of + e) = o;
    }
    for (int r = tid; r < QS; r += C::NT) {
      const int pos = cur.p0 + r;
      const bool ok = pos < si.len;
      const int64_t at = (int64_t)cur.hq * p.total_q + si.q0 + pos;
      lse_s[r] = ok ? st_lse[at] : INFINITY;  // padding rows: P = 0
      dl_s[r] = ok ? st_delta[at] : 0.f;
    }
    __syncthreads();
    const bool kvalid = kok && (!ku.causal_main || key < si.mainlen);
#pragma unroll 4
    for (int r = 0; r < QS; ++r) {
      float sdot = 0.f, pdot = 0.f;
#pragma unroll
      for (int d = 0; d < C::DPT; d += 4) {
        const float4 q4 = *(const float4*)(Qf + r * D + d0 + d);
        const float4 o4 = *(const float4*)(Of + r * D + d0 + d);
        sdot += q4.x * kf[d] + q4.y * kf[d + 1] + q4.z * kf[d + 2] + q4.w * kf[d + 3];
        pdot += o4.x * vf[d] + o4.y * vf[d + 1] + o4.z * vf[d + 2] + o4.w * vf[d + 3];
      }
      sdot = row_sum<C::TPR>(sdot);
      pdot = row_sum<C::TPR>(pdot);
      const float pv = kvalid ? fast_exp2(fmaf(sdot, c, -lse_s[r])) : 0.f;
      const float ds = pv * (pdot - dl_s[r]) * p.scale;
#pragma unroll
      for (int d = 0; d < C::DPT; d += 4) {
        const float4 q4 = *(const float4*)(Qf + r * D + d0 + d);
        const float4 o4 = *(const float4*)(Of + r * D + d0 + d);
        dk[d] += ds * q4.x, dk[d + 1] += ds * q4.y, dk[d + 2] += ds * q4.z, dk[d + 3] += ds * q4.w;
        dv[d] += pv * o4.x, dv[d + 1] += pv * o4.y, dv[d + 2] += pv * o4.z, dv[d + 3] += pv * o4.w;
      }
    }
  }
  if (!kok) return;
  if (mla) {  // V is K
#pragma unroll
    for (int d = 0; d < C::DPT; ++d) dk[d] += dv[d];
  }
  if (s.pages) {  // float32 gradients, added atomically
    float* dkf = (float*)s.dk + key_elem(s, s.dkbase, s.dksn, key) + d0;
    float* dvf = (float*)s.dv + key_elem(s, s.dvbase, s.dvsn, key) + d0;
#pragma unroll
    for (int d = 0; d < C::DPT; ++d) {
      atomicAdd(dkf + d, dk[d]);
      if (!mla) atomicAdd(dvf + d, dv[d]);
    }
    return;
  }
  T* dkp = (T*)s.dk + s.dkbase + (int64_t)key * s.dksn + d0;
  T* dvp = (T*)s.dv + s.dvbase + (int64_t)key * s.dvsn + d0;
#pragma unroll
  for (int d = 0; d < C::DPT; ++d) {
    dkp[d] = (T)dk[d];
    if (!mla) dvp[d] = (T)dv[d];
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct BwdFns {
  const void* dq;
  const void* dkv[2];  // main keys per sequence / causal token range (+ context)
  int dq_lds, dkv_lds, bq, dkv_keys;
  const void* dq_lse = nullptr;  // the dq kernel that reads the forward's row statistics
};

template <typename T, int D>
static BwdFns bwd_fns() {
  typedef BwdCfg<D> C;
  BwdFns f{(const void*)attn_bwd_dq_kernel<T, D, false>,
           {(const void*)attn_bwd_dkv_kernel<T, D, false>, (const void*)attn_bwd_dkv_kernel<T, D, true>},
           C::DQ_LDS,
           C::DKV_LDS,
           C::BQ,
           C::DKV_KEYS};
  // not for the 512-wide latent: at one wave per SIMD its allocation without the running
  // max (208 VGPRs + 144 AGPRs against 256 + 218) ran 14% slower
  if constexpr (!C::MLA_ONLY) f.dq_lse = (const void*)attn_bwd_dq_kernel<T, D, true>;
  return f;
}

template <typename T, int D>
static BwdFns bwd_simt_fns() {
  typedef SimtBwdCfg<D> C;
  return BwdFns{(const void*)attn_bwd_dq_simt_kernel<T, D>,
                {(const void*)attn_bwd_dkv_simt_kernel<T, D, false>, (const void*)attn_bwd_dkv_simt_kernel<T, D, true>},
                C::DQ_LDS,
                C::DKV_LDS,
                C::R,
                C::R};
}

// SIMT kernels: fp32, and head dims or modes without an MFMA backward
template <typename T>
static bool pick_bwd_simt(int D, BwdFns& f) {
  switch (D) {
    case 16: f = bwd_simt_fns<T, 16>(); return true;
    case 32: f = bwd_simt_fns<T, 32>(); return true;
    case 64: f = bwd_simt_fns<T, 64>(); return true;
    case 128: f = bwd_simt_fns<T, 128>(); return true;
    case 256: f = bwd_simt_fns<T, 256>(); return true;
    case 512: f = bwd_simt_fns<T, 512>(); return true;
    default: return false;
  }
}

template <typename T>
static bool pick_bwd(int D, BwdFns& f) {
  switch (D) {
    case 32: f = bwd_fns<T, 32>(); return true;
    case 64: f = bwd_fns<T, 64>(); return true;
    case 128: f = bwd_fns<T, 128>(); return true;
    case 256: f = bwd_fns<T, 256>(); return true;
    case 512: f = bwd_fns<T, 512>(); return true;  // MLA latent only (checked by the caller)
    default: return false;
  }
}

static int raise_lds(const void* fn, int bytes) {
  if (bytes <= 65536) return 0;
  static std::mutex mu;
  static const void* done[32];
  static int n_done = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_done; ++i)
    if (done[i] == fn) return 0;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return (int)e;
  if (n_done < 32) done[n_done++] = fn;
  return 0;
}

static bool row_ok(const void* ptr, int64_t sb, int64_t sh, int64_t sn) {
  // 16-byte aligned rows: base and every row stride a multiple of 8 elements
  return ((uintptr_t)ptr % 16 == 0) && sb % 8 == 0 && sh % 8 == 0 && sn % 8 == 0 && sn >= 0 &&
         sn < (1 << 22);
}

static int check_bwd(const fmlm_attn_params& p, const fmlm_attn_grads& g, BwdFns& f) {
  if (p.B < 0 || p.H < 0 || p.N < 0 || p.total_q < 0 || p.ctx_len < 0) return FMLM_E_ARG;
  const bool mla = p.flags & FMLM_FLAG_MLA;
  if (!p.q || !p.o || !p.k || (!mla && !p.v) || !g.dout || !g.dq || !g.dk || (!mla && !g.dv)) return FMLM_E_ARG;
  // MFMA kernels for bf16 / f16 (the 512-wide one only for the MLA latent), SIMT otherwise
  const bool mfma_ok = p.D != 16 && (p.D != 512 || mla);
  bool picked = false;
  if (p.dtype == FMLM_DTYPE_BF16) {
    picked = mfma_ok ? pick_bwd<bf16>(p.D, f) : pick_bwd_simt<bf16>(p.D, f);
  } else if (p.dtype == FMLM_DTYPE_F16) {
    picked = mfma_ok ? pick_bwd<f16>(p.D, f) : pick_bwd_simt<f16>(p.D, f);
  } else if (p.dtype == FMLM_DTYPE_F32) {
    picked = pick_bwd_simt<float>(p.D, f);
  } else {
    return FMLM_E_DTYPE;
  }
  if (!picked) return FMLM_E_HEAD_DIM;
  const bool causal = p.flags & FMLM_FLAG_CAUSAL_SEQ;
  if (causal && (!p.cu_seqlens_q || p.kv_layout != FMLM_LAYOUT_PACKED)) return FMLM_E_ARG;
  if (p.ctx_block_table && (p.ctx_pages_per_batch < 0 || p.ctx_rows < 1 || p.ctx_page_stride < 0))
    return FMLM_E_ARG;
  // keys shared by all heads must be shared by K and V alike
  if (!mla && ((p.k_sh == 0) != (p.v_sh == 0))) return FMLM_E_ARG;
  if (!row_ok(p.q, p.q_sb, p.q_sh, p.q_sn) || !row_ok(p.o, p.o_sb, p.o_sh, p.o_sn) ||
      !row_ok(p.k, p.k_sb, p.k_sh, p.k_sn) || (!mla && !row_ok(p.v, p.v_sb, p.v_sh, p.v_sn)) ||
      !row_ok(g.dout, g.do_sb, g.do_sh, g.do_sn) || !row_ok(g.dq, g.dq_sb, g.dq_sh, g.dq_sn) ||
      !row_ok(g.dk, g.dk_sb, g.dk_sh, g.dk_sn) || (!mla && !row_ok(g.dv, g.dv_sb, g.dv_sh, g.dv_sn)))
    return FMLM_E_ALIGN;
  // the gradients of shared keys are shared too
  if ((p.k_sh == 0) != (g.dk_sh == 0) || (!mla && (p.v_sh == 0) != (g.dv_sh == 0))) return FMLM_E_ARG;
  if (g.dk_ctx) {
    if (!p.k_ctx || (!mla && (!p.v_ctx || !g.dv_ctx))) return FMLM_E_ARG;
    if (!row_ok(p.k_ctx, p.c_sb, p.c_sh, p.c_sn) || !row_ok(g.dk_ctx, p.c_sb, p.c_sh, p.c_sn) ||
        (!mla && (!row_ok(p.v_ctx, p.c_sb, p.c_sh, p.c_sn) || !row_ok(g.dv_ctx, p.c_sb, p.c_sh, p.c_sn))))
      return FMLM_E_ALIGN;
    if ((p.cu_seqlens_kv || p.ctx_index) && p.ctx_batch < 1) return FMLM_E_ARG;
  }
  return 0;
}

}  // namespace
}  // namespace fmlm

using namespace fmlm;

// Units of the two grids and the workspace layout: the row statistics (2 H total_q
// floats), the sequence order and the unit tables (ints, see UnitTables), then the query
// and the key unit records (kRecInts ints each, 64-byte aligned).  bq, bk: query rows and
// keys per unit; n_ctx: context batches with gradients.
constexpr int kMinUnitRows = 16;  // the smallest bq / bk of any kernel pair
struct BwdLayout {
  int64_t qunits, kunits;  // units of the dq and of the dK / dV grid
  int64_t qrec, krec;      // byte offsets of their records
  int64_t bytes;
};
static BwdLayout bwd_layout(const fmlm_attn_params& p, int bq, int bk, int n_ctx) {
  BwdLayout l;
  const bool causal = p.flags & FMLM_FLAG_CAUSAL_SEQ;
  // at most total_q / bq + B query tiles; main keys: tiles per sequence, or of the causal
  // token range
  l.qunits = (int64_t)p.total_q / bq + p.B;
  const int64_t munits = causal ? ((int64_t)p.total_q + bk - 1) / bk : (int64_t)p.total_q / bk + p.B;
  // context rows over all batches: a packed context's rows per head, a paged one's pages
  // per batch (ctx_rows counts pool pages there), or the uniform length per batch
  const int64_t crows = n_ctx == 0            ? 0
                        : p.ctx_block_table   ? (int64_t)n_ctx * std::max(p.ctx_pages_per_batch, 0) * FMLM_PAGE_ROWS
                        : p.cu_seqlens_kv     ? (int64_t)std::max(p.ctx_rows, 0)
                                              : (int64_t)n_ctx * std::max(p.ctx_len, 0);
  l.kunits = munits + (n_ctx > 0 ? crows / bk + n_ctx : 0);
  const int64_t tables = 2 * (int64_t)p.H * p.total_q * 4 +
                         4 * ((int64_t)p.B + 2 * ((int64_t)p.B + 1) + (p.ctx_batch > 1 ? p.ctx_batch : 1) + 1);
  l.qrec = (tables + 63) / 64 * 64;
  l.krec = l.qrec + l.qunits * kRecInts * 4;
  l.bytes = (l.krec + l.kunits * kRecInts * 4 + 255) / 256 * 256;
  return l;
}

// The grid of `units` units x `heads` heads (grid_unit: heads fastest), at most 2^23
// workgroups per row; false if it has 2^31 workgroups or more.
static bool unit_grid(int64_t units, unsigned heads, dim3& grid) {
  if (units < 1 || heads < 1 || units * heads >= ((int64_t)1 << 31)) return false;
  const int64_t ux = std::min<int64_t>(units, std::max<int64_t>(1, ((int64_t)1 << 23) / heads));
  grid = dim3((unsigned)(ux * heads), (unsigned)((units + ux - 1) / ux));
  return true;
}

extern "C" int fmlm_attn_grads_size(void) { return (int)sizeof(fmlm_attn_grads); }

extern "C" int64_t fmlm_attn_bwd_workspace_bytes(const fmlm_attn_params* p) {
  if (!p || p->H < 0 || p->total_q < 0 || p->B < 0 || p->ctx_batch < 0) return FMLM_E_ARG;
  // every kernel pair's units have at least kMinUnitRows rows, and context gradients may
  // be asked for whenever there is a context
  const int n_ctx = p->k_ctx && !(p->flags & FMLM_FLAG_PREFILL) ? (p->ctx_batch > 1 ? p->ctx_batch : 1) : 0;
  return bwd_layout(*p, kMinUnitRows, kMinUnitRows, n_ctx).bytes;
}

extern "C" int fmlm_attn_bwd(const fmlm_attn_params* pp, const fmlm_attn_grads* gp, void* stream) {
  if (!pp || !gp) return FMLM_E_ARG;
  const fmlm_attn_params& p = *pp;
  const fmlm_attn_grads& g = *gp;
  BwdFns f;
  int rc = check_bwd(p, g, f);
  if (rc) return rc;
  if (p.B == 0 || p.H == 0 || p.total_q == 0) return 0;
  if (p.H > 65535) return FMLM_E_ARG;
  const bool prefill = p.flags & FMLM_FLAG_PREFILL;
  const bool causal = p.flags & FMLM_FLAG_CAUSAL_SEQ;
  const bool ctx_grads = g.dk_ctx && !prefill && p.k_ctx;
  int n_ctx = ctx_grads ? (p.ctx_batch > 1 ? p.ctx_batch : 1) : 0;
  const BwdLayout l = bwd_layout(p, f.bq, f.dkv_keys, n_ctx);
  if (!g.workspace || g.workspace_bytes < fmlm_attn_bwd_workspace_bytes(pp) || g.workspace_bytes < l.bytes)
    return FMLM_E_WORKSPACE;
  dim3 qgrid, kgrid;
  if (!unit_grid(l.qunits, (unsigned)p.H, qgrid) || !unit_grid(l.kunits, dkv_heads(p, n_ctx), kgrid)) return FMLM_E_ARG;
  hipStream_t s = (hipStream_t)stream;
  fmlm_attn_params pc = p;
  fmlm_attn_grads gc = g;
  int32_t* qrec = (int32_t*)((char*)g.workspace + l.qrec);
  int32_t* krec = (int32_t*)((char*)g.workspace + l.krec);
  int nq = (int)l.qunits, nk = (int)l.kunits;

  // 0. unit tables, then the records of both grids' units
  hipLaunchKernelGGL(bwd_units_kernel, dim3(1), dim3(kScanThreads), 0, s, p, g, f.bq, f.dkv_keys, n_ctx);
  if ((rc = launch_status())) return rc;
  const int64_t nrec = std::max(l.qunits, l.kunits);
  hipLaunchKernelGGL(bwd_records_kernel, dim3((unsigned)((nrec + 255) / 256)), dim3(256), 0, s, p, g, f.bq, f.dkv_keys,
                     n_ctx, qrec, nq, krec, nk);
  if ((rc = launch_status())) return rc;
  // 1. dq (+ the row statistics: delta, and the log2-sum-exp unless the forward stored it)
  const void* const dq_fn = p.lse && f.dq_lse ? f.dq_lse : f.dq;
  if ((rc = raise_lds(dq_fn, f.dq_lds))) return rc;
  void* args[] = {(void*)&pc, (void*)&gc, (void*)&qrec, (void*)&nq};
  hipError_t e = hipLaunchKernel(dq_fn, qgrid, dim3(kBwdNW * 64), args, (size_t)f.dq_lds, s);
  if (e != hipSuccess) return (int)e;
  // 2. dK / dV, context keys then main keys in one launch
  void* kargs[] = {(void*)&pc, (void*)&gc, (void*)&n_ctx, (void*)&krec, (void*)&nk};
  if ((rc = raise_lds(f.dkv[causal ? 1 : 0], f.dkv_lds))) return rc;
  e = hipLaunchKernel(f.dkv[causal ? 1 : 0], kgrid, dim3(kBwdNW * 64), kargs, (size_t)f.dkv_lds, s);
  if (e != hipSuccess) return (int)e;
  return launch_status();
}
