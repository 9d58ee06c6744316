// Fused non-causal MLM attention over [cached context || main keys] for gfx950.
//
// Semantics follow the reference device bodies:
//   _mlm_inner_attention        mlm_kernel_impl.py:10-62   (online softmax, exp2, P cast before P.V)
//   _mlm_main_kernel_impl       mlm_kernel_impl.py:65-216  (dense [B,H,N,D] addressing)
//   _mlm_compressed_kernel_impl mlm_kernel_impl.py:219-390 (packed varlen, context ranges,
//                                                          causal_query_seq_attn, MLA, prefill)
//
// Kernel design (bf16 / fp16):
//   * one workgroup = NW wave64s = one (query tile of BQ = NW*QB*16 rows, head);
//     each wave owns QB blocks of 16 query rows, held in registers as MFMA B operands.
//   * K/V tiles of BK keys are staged through LDS: K row-major [BK][D+8], V transposed
//     [D][BK+8] with a key permutation that makes each lane's eight P.V keys contiguous.
//     The next tile's global loads are issued before the current tile's math.
//   * S^T = K Q^T with v_mfma_f32_16x16x32_{bf16,f16}: the accumulator lane (q + 16g)
//     holds keys 4g..4g+3 of query q, so each lane owns one query row; softmax row
//     max/sum need two cross-lane steps (xor 16, xor 32).
//   * O^T = V^T P^T with the same instruction; the accumulator again keeps one query
//     per lane, so the online-softmax rescale is lane-local.
//   * fp32 accumulation, exp2 with scale*log2(e) folded, P rounded to the input type.
// The fp32 path (and head dims without an MFMA instantiation) uses a SIMT kernel with
// the same addressing.
#include "fmlm_common.h"

#include <mutex>

namespace fmlm {

// ---------------------------------------------------------------------------
// Work schedule: one item per (sequence b, query tile j) with tiles of BQ rows,
// only over real (unpadded) rows.
// ---------------------------------------------------------------------------
constexpr int kSchedThreads = 1024;

__global__ __launch_bounds__(kSchedThreads) void schedule_kernel(const int32_t* __restrict__ cu,
                                                                 int B, int BQ, int capacity,
                                                                 int2* __restrict__ items,
                                                                 int32_t* __restrict__ n_items) {
  __shared__ int s_til[kSchedThreads];
  const int tid = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < B; base += kSchedThreads) {
    const int b = base + tid;
    int tiles = 0;
    if (b < B) {
      const int len = cu[b + 1] - cu[b];
      tiles = len > 0 ? (len + BQ - 1) / BQ : 0;
    }
    s_til[tid] = tiles;
    __syncthreads();
    for (int off = 1; off < kSchedThreads; off <<= 1) {
      int t = tid >= off ? s_til[tid - off] : 0;
      __syncthreads();
      s_til[tid] += t;
      __syncthreads();
    }
    const int first = carry + s_til[tid] - tiles;
    for (int j = 0; j < tiles && first + j < capacity; ++j) items[first + j] = make_int2(b, j);
    carry += s_til[kSchedThreads - 1];
    __syncthreads();
  }
  if (tid == 0) *n_items = min(carry, capacity);
}

// ---------------------------------------------------------------------------
// Per-workgroup problem description resolved from (item, head).
// ---------------------------------------------------------------------------
struct KvSeg {
  const char* k;
  const char* v;
  int64_t kbase, vbase;  // element offset of key 0, or the head offset when lookup
  int64_t ksn, vsn;      // row strides
  int64_t ksb, vsb;      // sequence strides (lookup only)
  int n;                 // number of keys
  bool lookup;           // keys are packed token indices over a padded tensor
};

struct WorkItem {
  int b, h;
  int qpos0, qcount;     // query positions [qpos0, qpos0+qcount) of sequence b
  int64_t q_row0, o_row0;  // element offset of row qpos0
  int64_t q_sn, o_sn;
  KvSeg seg[2];          // context, main
};

FMLM_DEV int64_t seg_row(const KvSeg& s, int i, bool is_v, const int32_t* cu, int B) {
  const int64_t base = is_v ? s.vbase : s.kbase;
  const int64_t sn = is_v ? s.vsn : s.ksn;
  if (!s.lookup) return base + (int64_t)i * sn;
  const int bb = find_seq(cu, B, i);
  const int64_t sb = is_v ? s.vsb : s.ksb;
  return base + (int64_t)bb * sb + (int64_t)(i - cu[bb]) * sn;
}

// Resolve the workgroup's item.  Returns false for an idle workgroup.
FMLM_DEV bool resolve_work(const fmlm_attn_params& p, const int2* items, const int32_t* n_items,
                           int BQ, int esz, WorkItem& w) {
  int b, tile;
  if (p.cu_seqlens_q) {
    if ((int)blockIdx.x >= *n_items) return false;
    const int2 it = items[blockIdx.x];
    b = it.x;
    tile = it.y;
  } else {
    const int nt = (p.N + BQ - 1) / BQ;
    b = blockIdx.x / nt;
    tile = blockIdx.x % nt;
  }
  const int h = blockIdx.y;
  const int32_t* cu = p.cu_seqlens_q;
  const int q0 = seq_start(cu, b, p.N);
  int L = p.N;
  if (cu) {
    L = cu[b + 1] - q0;
    if (p.N > 0) L = min(L, p.N);
    L = max(min(L, p.total_q - q0), 0);
  }
  w.b = b;
  w.h = h;
  w.qpos0 = tile * BQ;
  w.qcount = min(BQ, L - w.qpos0);
  if (w.qcount <= 0) return false;
  const int64_t qb = p.q_layout == FMLM_LAYOUT_PACKED ? (int64_t)h * p.q_sh + (int64_t)q0 * p.q_sn
                                                      : (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const int64_t ob = p.o_layout == FMLM_LAYOUT_PACKED ? (int64_t)h * p.o_sh + (int64_t)q0 * p.o_sn
                                                      : (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
  w.q_row0 = qb + (int64_t)w.qpos0 * p.q_sn;
  w.o_row0 = ob + (int64_t)w.qpos0 * p.o_sn;
  w.q_sn = p.q_sn;
  w.o_sn = p.o_sn;
  const bool mla = p.flags & FMLM_FLAG_MLA;

  // context segment (mlm_kernel_impl.py:297-313 packed, :132-141 dense)
  KvSeg& c = w.seg[0];
  c.k = (const char*)p.k_ctx;
  c.v = (const char*)(mla ? p.k_ctx : p.v_ctx);
  c.lookup = false;
  c.n = 0;
  if (!(p.flags & FMLM_FLAG_PREFILL)) {
    const int cb = p.ctx_batch > 1 ? b : 0;
    int c0 = 0, c1 = p.ctx_len;
    if (p.cu_seqlens_kv) {
      c0 = min(max(p.cu_seqlens_kv[cb], 0), p.ctx_rows);
      c1 = min(max(p.cu_seqlens_kv[cb + 1], c0), p.ctx_rows);
    }
    c.n = max(c1 - c0, 0);
    c.kbase = (int64_t)cb * p.c_sb + (int64_t)h * p.c_sh + (int64_t)c0 * p.c_sn;
    c.vbase = c.kbase;
    c.ksn = c.vsn = p.c_sn;
    c.ksb = c.vsb = 0;
  }
  // main segment (mlm_kernel_impl.py:288-293, 360-379)
  KvSeg& m = w.seg[1];
  m.k = (const char*)p.k;
  m.v = (const char*)(mla ? p.k : p.v);
  const int64_t v_sb = mla ? p.k_sb : p.v_sb, v_sh = mla ? p.k_sh : p.v_sh,
                v_sn = mla ? p.k_sn : p.v_sn;
  m.ksn = p.k_sn;
  m.vsn = v_sn;
  m.ksb = p.k_sb;
  m.vsb = v_sb;
  const bool causal = (p.flags & FMLM_FLAG_CAUSAL_SEQ) && cu;
  if (causal) {
    m.n = q0 + L;  // packed tokens [0, cu[b+1])
    m.kbase = (int64_t)h * p.k_sh;
    m.vbase = (int64_t)h * v_sh;
    m.lookup = p.kv_layout != FMLM_LAYOUT_PACKED;
  } else {
    m.n = L;
    m.lookup = false;
    if (p.kv_layout == FMLM_LAYOUT_PACKED) {
      m.kbase = (int64_t)h * p.k_sh + (int64_t)q0 * p.k_sn;
      m.vbase = (int64_t)h * v_sh + (int64_t)q0 * v_sn;
    } else {
      m.kbase = (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
      m.vbase = (int64_t)b * v_sb + (int64_t)h * v_sh;
    }
  }
  (void)esz;
  return true;
}

FMLM_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// MFMA kernel (bf16 / fp16)
// ---------------------------------------------------------------------------
template <typename T>
struct Mfma;
template <>
struct Mfma<bf16> {
  typedef bf16x8 v8;
  static FMLM_DEV f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<f16> {
  typedef f16x8 v8;
  static FMLM_DEV f32x4 run(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Position of key k (within a BK tile) in the transposed V tile.  Within each
// 32-key block, key 16*hf + 4*g + r goes to 8*g + 4*hf + r so that lane group g
// reads its eight P.V keys (the S^T rows 4g..4g+3 of two adjacent 16-key blocks)
// as one 16-byte row segment.
FMLM_DEV int vt_pos(int k) {
  const int blk = k >> 5, kk = k & 31;
  const int hf = kk >> 4, g = (kk >> 2) & 3, r = kk & 3;
  return (blk << 5) + (g << 3) + (hf << 2) + r;
}

template <typename T, int D, int QB, int NW, int BK>
struct MfmaCfg {
  static constexpr int NT = NW * 64;
  static constexpr int BQ = NW * QB * 16;
  static constexpr int KS = D + 8;   // LDS K row stride (elements)
  static constexpr int VS = BK + 8;  // LDS V^T row stride (elements)
  static constexpr int KTILE = BK * KS;
  static constexpr int VTILE = D * VS;
  static constexpr int LDS_BYTES = (KTILE + VTILE) * 2;
  static constexpr int KC = (D + 31) / 32;   // 32-wide contraction steps over D
  static constexpr int NDB = D / 16;         // 16-wide output column blocks
  static constexpr int NKB = BK / 16;        // 16-key S^T blocks per tile
  static constexpr int NKS = BK / 32;        // 32-key P.V steps per tile
  static constexpr int C8 = D / 8;           // 16-byte chunks per row
  static constexpr int LITEMS = (BK / 4) * C8;  // loader items (4 keys x 8 columns)
  static constexpr int LPT = (LITEMS + NT - 1) / NT;  // loader items per thread
  static_assert(D % 16 == 0 && D >= 16, "head dim");
  static_assert(BK % 32 == 0, "key tile");
};

template <typename T, int D, int QB, int NW, int BK>
__global__ __launch_bounds__(NW * 64) void attn_mfma_kernel(const fmlm_attn_params p,
                                                            const int2* __restrict__ items,
                                                            const int32_t* __restrict__ n_items) {
  typedef MfmaCfg<T, D, QB, NW, BK> C;
  typedef typename Mfma<T>::v8 v8;
  extern __shared__ __align__(16) char smem_raw[];
  T* Ks = (T*)smem_raw;
  T* Vt = Ks + C::KTILE;

  WorkItem w;
  if (!resolve_work(p, items, n_items, C::BQ, 2, w)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int32_t* cu = p.cu_seqlens_q;
  const int B = p.B;

  // ---- Q fragments: lane (q + 16g), block qb, step kc holds Q[row][kc*32 + 8g .. +8]
  v8 qf[QB][C::KC];
  const char* qbase = (const char*)p.q;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = (wave * QB + qb) * 16 + l16;
    const bool ok = row < w.qcount;
    const int64_t off = w.q_row0 + (int64_t)row * w.q_sn;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      const int col = kc * 32 + g * 8;
      if (ok && col < D)
        qf[qb][kc] = *(const v8*)(qbase + (off + col) * 2);
      else
        qf[qb][kc] = v8{};
    }
  }

  f32x4 o[C::NDB][QB];
#pragma unroll
  for (int db = 0; db < C::NDB; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i[QB], l_i[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = -INFINITY;
    l_i[qb] = 0.f;
  }
  const float c = p.scale * kLog2e;

  // ---- tile sequence: context tiles then main tiles
  const int nt0 = (w.seg[0].n + BK - 1) / BK;
  const int nt1 = (w.seg[1].n + BK - 1) / BK;
  const int ntiles = nt0 + nt1;

  u32x4 kreg[C::LPT][4], vreg[C::LPT][4];
  auto issue_loads = [&](int t) {
    const KvSeg& s = t < nt0 ? w.seg[0] : w.seg[1];
    const int j0 = (t < nt0 ? t : t - nt0) * BK;
#pragma unroll
    for (int li = 0; li < C::LPT; ++li) {
      const int it = tid + li * C::NT;
      const int kq = it / C::C8, c8 = it % C::C8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = j0 + kq * 4 + r;
        if (it < C::LITEMS && key < s.n) {
          const int64_t kr = seg_row(s, key, false, cu, B);
          const int64_t vr = seg_row(s, key, true, cu, B);
          kreg[li][r] = *(const u32x4*)(s.k + (kr + c8 * 8) * 2);
          vreg[li][r] = *(const u32x4*)(s.v + (vr + c8 * 8) * 2);
        } else {
          kreg[li][r] = u32x4{0u, 0u, 0u, 0u};
          vreg[li][r] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  };
  auto store_lds = [&]() {
#pragma unroll
    for (int li = 0; li < C::LPT; ++li) {
      const int it = tid + li * C::NT;
      if (it >= C::LITEMS) continue;
      const int kq = it / C::C8, c8 = it % C::C8;
#pragma unroll
      for (int r = 0; r < 4; ++r) *(u32x4*)(Ks + (kq * 4 + r) * C::KS + c8 * 8) = kreg[li][r];
      // transpose 4 keys x 8 columns into 8 rows of V^T (4 keys each)
      const int pos = vt_pos(kq * 4);
#pragma unroll
      for (int dw = 0; dw < 4; ++dw) {
        const uint32_t a0 = vreg[li][0][dw], a1 = vreg[li][1][dw];
        const uint32_t a2 = vreg[li][2][dw], a3 = vreg[li][3][dw];
        u32x2 lo, hi;
        lo[0] = (a0 & 0xffffu) | (a1 << 16);
        lo[1] = (a2 & 0xffffu) | (a3 << 16);
        hi[0] = (a0 >> 16) | (a1 & 0xffff0000u);
        hi[1] = (a2 >> 16) | (a3 & 0xffff0000u);
        *(u32x2*)(Vt + (c8 * 8 + dw * 2) * C::VS + pos) = lo;
        *(u32x2*)(Vt + (c8 * 8 + dw * 2 + 1) * C::VS + pos) = hi;
      }
    }
  };

  if (ntiles > 0) issue_loads(0);
  for (int t = 0; t < ntiles; ++t) {
    const int nk = t < nt0 ? min(BK, w.seg[0].n - t * BK) : min(BK, w.seg[1].n - (t - nt0) * BK);
    __syncthreads();  // previous tile's LDS reads are done
    store_lds();
    __syncthreads();
    if (t + 1 < ntiles) issue_loads(t + 1);

    // ---- S^T = K Q^T
    f32x4 s[C::NKB][QB];
#pragma unroll
    for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      const int col = kc * 32 + g * 8;
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
        v8 a = col < D ? *(const v8*)(Ks + (kb * 16 + l16) * C::KS + col) : v8{};
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[kb][qb] = Mfma<T>::run(a, qf[qb][kc], s[kb][qb]);
      }
    }

    // ---- online softmax (mlm_kernel_impl.py:42-60); lane owns query l16 of each block
    const bool partial = nk < BK;
    typename Mfma<T>::v8 pf[C::NKS][QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (partial) {
#pragma unroll
        for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (kb * 16 + g * 4 + r >= nk) s[kb][qb][r] = -INFINITY;
      }
      float mx = -INFINITY;
      if (c >= 0.f) {
#pragma unroll
        for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kb][qb][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        mx *= c;
      } else {
        float mn = INFINITY;
#pragma unroll
        for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            mn = s[kb][qb][r] == -INFINITY ? mn : fminf(mn, s[kb][qb][r]);
        mn = fminf(mn, __shfl_xor(mn, 16));
        mn = fminf(mn, __shfl_xor(mn, 32));
        mx = mn * c;
      }
      const float m_new = fmaxf(m_i[qb], mx);
      const float alpha = fast_exp2(m_i[qb] - m_new);
      m_i[qb] = m_new;
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = s[kb][qb][r];
          const float pv = x == -INFINITY ? 0.f : fast_exp2(x * c - m_new);
          rs += pv;
          pf[kb >> 1][qb][(kb & 1) * 4 + r] = (T)pv;
        }
      }
      l_i[qb] = l_i[qb] * alpha + rs;
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) o[db][qb] *= alpha;
    }

    // ---- O^T += V^T P^T
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        const v8 a = *(const v8*)(Vt + (db * 16 + l16) * C::VS + ks * 32 + g * 8);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[db][qb] = Mfma<T>::run(a, pf[ks][qb], o[db][qb]);
      }
    }
  }

  // ---- epilogue: O /= l (l == 0 -> 1), store valid rows (mlm_kernel_impl.py:381-390)
  char* obase = (char*)p.o;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    float l = l_i[qb];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = l > 0.f ? 1.f / l : 1.f;
    const int row = (wave * QB + qb) * 16 + l16;
    if (row >= w.qcount) continue;
    const int64_t off = w.o_row0 + (int64_t)row * w.o_sn;
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      T v4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = (T)(o[db][qb][r] * inv);
      *(u32x2*)(obase + (off + db * 16 + g * 4) * 2) = *(const u32x2*)v4;
    }
  }
}

// ---------------------------------------------------------------------------
// SIMT kernel: one query row per TPR threads (each holding D/TPR dims), K/V tiles
// staged in LDS as fp32.  Used for fp32 inputs and head dims without an MFMA
// instantiation.  Probabilities are rounded to T before P.V like the MFMA path.
// ---------------------------------------------------------------------------
template <int D>
struct SimtCfg {
  static constexpr int TPR = D > 64 ? D / 64 : 1;  // threads per query row
  static constexpr int DPT = D / TPR;              // dims per thread
  static constexpr int RPW = 64;                   // query rows per workgroup
  static constexpr int NT = RPW * TPR;
  static constexpr int BKS = (4096 / D) < 8 ? 8 : ((4096 / D) > 64 ? 64 : (4096 / D));
  static constexpr int LDS_BYTES = 2 * BKS * D * 4;
};

template <typename T>
FMLM_DEV float to_f(T x) {
  return (float)x;
}

template <typename T, int D>
__global__ __launch_bounds__(SimtCfg<D>::NT) void attn_simt_kernel(
    const fmlm_attn_params p, const int2* __restrict__ items, const int32_t* __restrict__ n_items) {
  typedef SimtCfg<D> C;
  extern __shared__ __align__(16) char smem_raw[];
  float* Kf = (float*)smem_raw;
  float* Vf = Kf + C::BKS * D;

  WorkItem w;
  if (!resolve_work(p, items, n_items, C::RPW, (int)sizeof(T), w)) return;
  const int tid = threadIdx.x;
  const int row = tid / C::TPR;
  const int part = tid % C::TPR;
  const int d0 = part * C::DPT;
  const int32_t* cu = p.cu_seqlens_q;
  const int B = p.B;
  const float c = p.scale * kLog2e;

  float q[C::DPT], o[C::DPT];
  const bool ok = row < w.qcount;
  const T* qp = (const T*)p.q + w.q_row0 + (int64_t)row * w.q_sn + d0;
#pragma unroll
  for (int d = 0; d < C::DPT; ++d) {
    q[d] = ok ? to_f(qp[d]) : 0.f;
    o[d] = 0.f;
  }
  float m_i = -INFINITY, l_i = 0.f;

  for (int si = 0; si < 2; ++si) {
    const KvSeg& s = w.seg[si];
    for (int j0 = 0; j0 < s.n; j0 += C::BKS) {
      const int nk = min(C::BKS, s.n - j0);
      __syncthreads();
      for (int e = tid; e < C::BKS * D; e += C::NT) {
        const int kk = e / D, d = e % D;
        float kv = 0.f, vv = 0.f;
        if (kk < nk) {
          const int64_t kr = seg_row(s, j0 + kk, false, cu, B);
          const int64_t vr = seg_row(s, j0 + kk, true, cu, B);
          kv = to_f(((const T*)s.k)[kr + d]);
          vv = to_f(((const T*)s.v)[vr + d]);
        }
        Kf[e] = kv;
        Vf[e] = vv;
      }
      __syncthreads();
      float sc[C::BKS];
      float mx = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < C::BKS; ++kk) {
        float acc = 0.f;
#pragma unroll
        for (int d = 0; d < C::DPT; ++d) acc += q[d] * Kf[kk * D + d0 + d];
#pragma unroll
        for (int off = 1; off < C::TPR; off <<= 1) acc += __shfl_xor(acc, off);
        sc[kk] = kk < nk ? acc * c : -INFINITY;
        mx = fmaxf(mx, sc[kk]);
      }
      const float m_new = fmaxf(m_i, mx);
      const float alpha = fast_exp2(m_i - m_new);
      m_i = m_new;
      l_i *= alpha;
#pragma unroll
      for (int d = 0; d < C::DPT; ++d) o[d] *= alpha;
#pragma unroll
      for (int kk = 0; kk < C::BKS; ++kk) {
        const float pv = kk < nk ? fast_exp2(sc[kk] - m_new) : 0.f;
        l_i += pv;
        const float pr = to_f((T)pv);
#pragma unroll
        for (int d = 0; d < C::DPT; ++d) o[d] += pr * Vf[kk * D + d0 + d];
      }
    }
  }
  if (!ok) return;
  const float inv = l_i > 0.f ? 1.f / l_i : 1.f;
  T* op = (T*)p.o + w.o_row0 + (int64_t)row * w.o_sn + d0;
#pragma unroll
  for (int d = 0; d < C::DPT; ++d) op[d] = (T)(o[d] * inv);
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
struct Launch {
  int bq;         // query rows per workgroup
  int threads;
  int lds;
  const void* fn;
};

template <typename T, int D, int QB, int NW, int BK>
static Launch mfma_launch() {
  typedef MfmaCfg<T, D, QB, NW, BK> C;
  return Launch{C::BQ, C::NT, C::LDS_BYTES, (const void*)&attn_mfma_kernel<T, D, QB, NW, BK>};
}

template <typename T, int D>
static Launch simt_launch() {
  typedef SimtCfg<D> C;
  return Launch{C::RPW, C::NT, C::LDS_BYTES, (const void*)&attn_simt_kernel<T, D>};
}

template <typename T>
static bool pick_mfma(int D, Launch& L) {
  switch (D) {
    case 16: L = mfma_launch<T, 16, 2, 4, 64>(); return true;
    case 32: L = mfma_launch<T, 32, 2, 4, 64>(); return true;
    case 64: L = mfma_launch<T, 64, 2, 4, 64>(); return true;
    case 128: L = mfma_launch<T, 128, 2, 4, 64>(); return true;
    case 256: L = mfma_launch<T, 256, 1, 4, 64>(); return true;
    default: return false;
  }
}

template <typename T>
static bool pick_simt(int D, Launch& L) {
  switch (D) {
    case 16: L = simt_launch<T, 16>(); return true;
    case 32: L = simt_launch<T, 32>(); return true;
    case 64: L = simt_launch<T, 64>(); return true;
    case 128: L = simt_launch<T, 128>(); return true;
    case 256: L = simt_launch<T, 256>(); return true;
    case 512: L = simt_launch<T, 512>(); return true;
    default: return false;
  }
}

static int pick_launch(int dtype, int D, Launch& L) {
  bool ok = false;
  switch (dtype) {
    case FMLM_DTYPE_BF16: ok = pick_mfma<bf16>(D, L) || pick_simt<bf16>(D, L); break;
    case FMLM_DTYPE_F16: ok = pick_mfma<f16>(D, L) || pick_simt<f16>(D, L); break;
    case FMLM_DTYPE_F32: ok = pick_simt<float>(D, L); break;
    default: return FMLM_E_DTYPE;
  }
  return ok ? 0 : FMLM_E_HEAD_DIM;
}

static int64_t max_items(const fmlm_attn_params& p, int bq) {
  if (!p.cu_seqlens_q) return (int64_t)p.B * ((p.N + bq - 1) / bq);
  return (int64_t)p.B + p.total_q / bq + 1;
}

static int64_t workspace_for(const fmlm_attn_params& p, int bq) {
  if (!p.cu_seqlens_q) return 0;
  return 256 + max_items(p, bq) * (int64_t)sizeof(int2);
}

static int check_params(const fmlm_attn_params& p) {
  if (p.B < 0 || p.H < 0 || p.N < 0 || p.D < 1 || p.total_q < 0 || p.ctx_len < 0) return FMLM_E_ARG;
  if (!p.q || !p.o || !p.k || (!(p.flags & FMLM_FLAG_MLA) && !p.v)) return FMLM_E_ARG;
  if ((p.flags & FMLM_FLAG_CAUSAL_SEQ) && !p.cu_seqlens_q) return FMLM_E_ARG;
  if (!(p.flags & FMLM_FLAG_PREFILL)) {
    const bool has_ctx = p.cu_seqlens_kv || p.ctx_len > 0;
    if (has_ctx && !p.cu_seqlens_kv && p.ctx_len > 0 && !p.k_ctx) return FMLM_E_ARG;
    if (p.cu_seqlens_kv && p.ctx_batch < 1) return FMLM_E_ARG;
  }
  return 0;
}

static int launch_schedule(const fmlm_attn_params& p, int bq, char* sched, hipStream_t s) {
  const int64_t cap = max_items(p, bq);
  if (cap > 0x7fffffff) return FMLM_E_ARG;
  hipLaunchKernelGGL(schedule_kernel, dim3(1), dim3(kSchedThreads), 0, s, p.cu_seqlens_q, p.B, bq,
                     (int)cap, (int2*)(sched + 256), (int32_t*)sched);
  return launch_status();
}

}  // namespace fmlm

using namespace fmlm;

extern "C" int fmlm_attn_schedule(const fmlm_attn_params* pp, void* schedule,
                                  int64_t schedule_bytes, void* stream) {
  if (!pp || !schedule || !pp->cu_seqlens_q || pp->B < 1) return FMLM_E_ARG;
  Launch L;
  const int rc = pick_launch(pp->dtype, pp->D, L);
  if (rc) return rc;
  if (schedule_bytes < workspace_for(*pp, L.bq)) return FMLM_E_WORKSPACE;
  return launch_schedule(*pp, L.bq, (char*)schedule, (hipStream_t)stream);
}

extern "C" int fmlm_attn_params_size(void) { return (int)sizeof(fmlm_attn_params); }

extern "C" int64_t fmlm_attn_workspace_bytes(const fmlm_attn_params* p) {
  if (!p) return FMLM_E_ARG;
  Launch L;
  const int rc = pick_launch(p->dtype, p->D, L);
  if (rc) return rc;
  return workspace_for(*p, L.bq);
}

extern "C" int fmlm_attn_fwd(const fmlm_attn_params* pp, void* stream) {
  if (!pp) return FMLM_E_ARG;
  const fmlm_attn_params& p = *pp;
  int rc = check_params(p);
  if (rc) return rc;
  Launch L;
  rc = pick_launch(p.dtype, p.D, L);
  if (rc) return rc;
  if (p.B == 0 || p.H == 0) return 0;
  const int64_t need = workspace_for(p, L.bq);
  if (need > 0 && !p.schedule && (!p.workspace || p.workspace_bytes < need)) return FMLM_E_WORKSPACE;
  if (p.H > 65535) return FMLM_E_ARG;
  hipStream_t s = (hipStream_t)stream;

  // allow > 64 KiB of dynamic LDS once per kernel
  {
    static std::mutex mu;
    static const void* raised[64];
    static int n_raised = 0;
    std::lock_guard<std::mutex> lock(mu);
    bool done = false;
    for (int i = 0; i < n_raised; ++i) done = done || raised[i] == L.fn;
    if (!done) {
      hipError_t e = hipFuncSetAttribute(L.fn, hipFuncAttributeMaxDynamicSharedMemorySize, L.lds);
      if (e != hipSuccess) return (int)e;
      if (n_raised < 64) raised[n_raised++] = L.fn;
    }
  }

  int2* items = nullptr;
  int32_t* n_items = nullptr;
  if (p.cu_seqlens_q) {
    char* sched = (char*)(p.schedule ? p.schedule : p.workspace);
    n_items = (int32_t*)sched;
    items = (int2*)(sched + 256);
    if (!p.schedule) {
      rc = launch_schedule(p, L.bq, sched, s);
      if (rc) return rc;
    }
  }
  const int64_t gx = max_items(p, L.bq);
  if (gx <= 0) return 0;
  if (gx > 0x7fffffff) return FMLM_E_ARG;
  fmlm_attn_params pc = p;
  void* args[] = {(void*)&pc, (void*)&items, (void*)&n_items};
  hipError_t e = hipLaunchKernel(L.fn, dim3((unsigned)gx, (unsigned)p.H), dim3(L.threads), args,
                                 (size_t)L.lds, s);
  if (e != hipSuccess) return (int)e;
  return launch_status();
}
