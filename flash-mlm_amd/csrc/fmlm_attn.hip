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

#include <algorithm>
#include <type_traits>
#include <mutex>

namespace fmlm {

// ---------------------------------------------------------------------------
// Work schedule.  A work unit is (sequence b, head h, query tile j) with tiles of BQ
// real (unpadded) rows.  Units of one (b, h) group share that group's K/V, and the
// groups of one head may share keys too (a shared context, the causal token range), so
// groups are kept on few XCDs: units meant for XCD x go to queue x, whose entries are
// run by workgroups the dispatcher hands to XCD x (workgroup w goes to XCD w % 8).  The
// groups of a head are cut into parts by sequence rank and each XCD takes a run of parts
// in head order (see schedule_kernel); within a part, groups go longest-first (estimated
// keys x tiles).
// The list is built once per cu_seqlens by schedule_kernel and cached by the host.
//
// Queues.  Queue x holds header[8 + x] units at units + x * cap (cap = header[5], a
// bound on the whole launch's units, so one queue never overflows whatever the
// placement).  A launch runs one unit per workgroup over G >= cap workgroups: workgroup
// w takes entry w / 8 of queue w % 8 (entries [0, G_x) of queue x, G_x = ceil((G - x) /
// 8), are taken this way, in dispatch order); a workgroup whose queue has no such entry
// is a spare and takes, by its rank among the spares, one of the entries past G_y of the
// queues y that hold more than G_y (see workgroup_unit).  Placements keep the queues
// about equally long, so overflow entries are few and most spares exit at once.
// Head-packed launches run 8 * cap workgroups (every entry its static workgroup's).
//
// Split-KV: when the units would fill the GPU's workgroup slots for fewer than
// kSplitRounds rounds, each query tile's key range is cut into S parts (a split group);
// every part is a unit that writes a partial record (O / l as fp32, then m and l per
// row) and a second kernel, merge_kernel, combines each group's records into the output.
// (Merging inside the attention kernel would need device-scope release/acquire between
// workgroups, which writes back and invalidates an XCD's whole L2 each time.)
//
// Unit encoding (int4): x = b, y = h | tile << 16, z = first record of the split group,
// w = -1 (no split) or group | s << 20 | (S - 1) << 25.
// Schedule buffer: [0, 256) header (units, n_groups, groups / records offsets, record
// bytes, queue capacity, queue lengths), the queues at 256, then the
// group list (int4: b, h | tile << 16, first record, S), then the records.
// ---------------------------------------------------------------------------
constexpr int kXcds = 8;
constexpr int kSchedThreads = 512;  // one wave per XCD
constexpr int kSortMax = 2048;      // sequences ordered longest-first up to this many
constexpr int kSplitBK = 64;        // key tile of the split-capable kernel
constexpr int kMaxSplits = 16;
constexpr int kMinSplitTiles = 8;   // key tiles per part at least
constexpr float kSplitRounds = 1.5f;
// schedule header fields (int32 index)
constexpr int kHdrUnits = 0;      // units in all queues
constexpr int kHdrGroups = 1;     // split groups
constexpr int kHdrGroupsOff = 2;  // byte offsets of the group list and the records
constexpr int kHdrRecordsOff = 3;
constexpr int kHdrRecBytes = 4;
constexpr int kHdrCap = 5;        // entries per queue
constexpr int kHdrQueueLen = 8;   // [8, 16): entries of queue x


__global__ __launch_bounds__(kSchedThreads) void schedule_kernel(const fmlm_attn_params p, int BQ,
                                                                 int cap_q, int slots,
                                                                 int rec_cap,
                                                                 int4* __restrict__ units,
                                                                 int32_t* __restrict__ header,
                                                                 int4* __restrict__ groups,
                                                                 int groups_off, int records_off,
                                                                 int rec_bytes, int hpack) {
  __shared__ int s_tiles[kSortMax];
  __shared__ int s_kt[kSortMax];            // key tiles per query tile
  __shared__ long long s_pre[kSortMax + 1];  // head-packed: work before each rank
  __shared__ float s_work[kSortMax];
  __shared__ int s_order[kSortMax];
  __shared__ unsigned char s_split[kSortMax];
  __shared__ int s_len[kXcds];
  __shared__ float s_sum[2];
  __shared__ int s_chunk, s_groups, s_recs;
  const int tid = threadIdx.x;
  const int B = p.B, H = p.H;
  const bool sorted = B <= kSortMax;
  // head-packed tiles (hpack, MLA): a tile is BQ consecutive rows of the H*L (head,
  // position) rows of a sequence, since every head reads the same latent.  The latent of a
  // sequence is larger than an XCD's L2, so a sequence's tiles go to as few XCDs as
  // possible: the sequences in rank order are laid end to end by work (tiles x key tiles),
  // the total is cut into kXcds equal parts, and each tile goes to the XCD whose part
  // holds its midpoint (a sequence spans one XCD, or two or three at the cuts).  Unsorted
  // batches deal tile t of every sequence to XCD t % kXcds.
  const int HG = hpack ? kXcds : H;  // groups per sequence
  auto seq_tiles = [&](int len) { return ((hpack ? H : 1) * len + BQ - 1) / BQ; };
  auto group_tiles = [&](int tiles, int j) { return hpack ? max(0, (tiles - j + kXcds - 1) / kXcds) : tiles; };
  if (tid < 2) s_sum[tid] = 0.f;
  if (tid == 0) {
    s_chunk = 0;
    s_groups = 0;
    s_recs = 0;
  }
  __syncthreads();
  if (sorted) {
    // per sequence: query tiles and key tiles; totals of units and key-tile work
    for (int b = tid; b < B; b += kSchedThreads) {
      const SeqInfo si = seq_info(p, b);
      const int tiles = seq_tiles(si.len);
      const int ktiles = (si.ctx + kSplitBK - 1) / kSplitBK + (si.mainlen + kSplitBK - 1) / kSplitBK;
      const float units = (float)tiles * (hpack ? 1 : H);
      s_tiles[b] = tiles;
      s_kt[b] = ktiles;
      s_work[b] = (float)ktiles;
      atomicAdd(&s_sum[0], units);
      atomicAdd(&s_sum[1], units * ktiles);
    }
    __syncthreads();
    // split only when the units are too few to fill the slots for kSplitRounds rounds;
    // parts of about total / (kSplitRounds * slots) key tiles, at least kMinSplitTiles,
    // the part size doubling until the records fit
    if (tid == 0 && rec_cap > 0 && s_sum[0] < kSplitRounds * slots) {
      int chunk = max(kMinSplitTiles, (int)ceilf(s_sum[1] / (kSplitRounds * slots)));
      for (int it = 0; it < 24; ++it, chunk *= 2) {
        float recs = 0.f;
        for (int b = 0; b < B; ++b) {
          const int S = min(kMaxSplits, max(1, (int)ceilf(s_work[b] / chunk)));
          if (S > 1) recs += (float)s_tiles[b] * (hpack ? 1 : H) * S;
        }
        if (recs <= (float)rec_cap) {
          s_chunk = chunk;
          break;
        }
      }
    }
    __syncthreads();
    for (int b = tid; b < B; b += kSchedThreads) {
      const int S = s_chunk > 0 ? min(kMaxSplits, max(1, (int)ceilf(s_work[b] / s_chunk))) : 1;
      s_split[b] = (unsigned char)S;
      // longest unit first (key tiles per part), then more tiles first
      s_work[b] = ceilf(s_work[b] / S) * 65536.f + (float)s_tiles[b];
    }
    __syncthreads();
    for (int b = tid; b < B; b += kSchedThreads) {
      const float wb = s_work[b];
      int rank = 0;
      for (int o = 0; o < B; ++o) {
        const float wo = s_work[o];
        rank += (wo > wb) || (wo == wb && o < b);
      }
      s_order[rank] = b;
    }
    __syncthreads();
    if (hpack && tid == 0) {  // work before each rank (a tile with no keys counts as one)
      long long acc = 0;
      for (int r = 0; r < B; ++r) {
        s_pre[r] = acc;
        const int b = s_order[r];
        acc += (long long)s_tiles[b] * max(s_kt[b], 1);
      }
      s_pre[B] = acc;
    }
    __syncthreads();
  }
  const int x = tid >> 6, lane = tid & 63;
  const int G = B * HG;
  // One tile per (sequence, head): the sequences of a head may share its keys (a shared
  // context, the causal token range), so the groups of a head stay on as few XCDs as
  // possible.  Head h's groups are cut into K = 8 / gcd(H, 8) parts by rank (rank block j,
  // ranks [jK, jK + K), gives part p rank jK + p for even j, jK + K - 1 - p for odd j,
  // which evens out the parts' work; longest first) and XCD x takes parts [x PX, (x + 1) PX) of the H K parts
  // in head order: every XCD gets PX parts, and a head's keys are read by ceil(8 / H)
  // XCDs or one more (at most two from 8 heads up).  (Head-packed tiles, and unsorted
  // batches, go round-robin: group g to XCD g % 8.)
  const bool by_head = sorted && !hpack;
  const bool by_seq = sorted && hpack;
  // by_seq: the first tile of rank r whose work midpoint lies at or past the start of
  // XCD x's part, i.e. 8 P_r + (8 i + 4) k >= x W
  auto first_tile = [&](int r, int xx) {
    const long long W = s_pre[B], k = max(s_kt[s_order[r]], 1);
    const long long num = (long long)xx * W - 8 * s_pre[r] - 4 * k;
    const long long i = num <= 0 ? 0 : (num + 8 * k - 1) / (8 * k);
    return (int)min(i, (long long)s_tiles[s_order[r]]);
  };
  const int K = kXcds / min(H & -H, kXcds);
  const int PX = H * K / kXcds;
  const int nrank = (B + K - 1) / K;
  int carry = 0;
  for (int i0 = 0; by_head ? i0 < PX * nrank : by_seq ? i0 < B : x + kXcds * i0 < G; i0 += 64) {
    bool valid;
    int r = 0;
    int b = 0, h = 0, tiles = 0, S = 1;
    int t0 = 0, tstep = kXcds;  // head-packed: the j-th tile of the group is t0 + tstep * j
    if (by_seq) {  // rank r's tiles in XCD x's part
      r = i0 + lane;
      valid = r < B;
    } else if (by_head) {  // this XCD's group i: part q = x PX + i / nrank, its (i % nrank)-th rank
      const int i = i0 + lane;
      const int q = x * PX + i / nrank, j = i % nrank, pq = q % K;
      h = q / K;
      r = j * K + ((j & 1) ? K - 1 - pq : pq);  // ranks dealt to the parts back and forth
      valid = i < PX * nrank && r < B;
    } else {
      const int g = x + kXcds * (i0 + lane);
      valid = g < G;
      r = g / HG;
      h = g - r * HG;
    }
    if (valid) {
      b = sorted ? s_order[r] : r;
      if (by_seq) {
        t0 = first_tile(r, x);
        tstep = 1;
        tiles = first_tile(r, x + 1) - t0;
      } else {
        t0 = h;
        tiles = group_tiles(sorted ? s_tiles[b] : seq_tiles(seq_info(p, b).len), h);
      }
      S = sorted ? s_split[b] : 1;
    }
    const int n = tiles * S;
    // inclusive wave scan of units
    int incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off);
      if (lane >= off) incl += v;
    }
    const int pos = carry + incl - n;
    int gid0 = 0, rec0 = 0;
    // (h, tile) field of the unit: head-packed tiles carry no head
    auto hf = [&](int j) { return hpack ? ((t0 + tstep * j) << 16) : (h | (j << 16)); };
    if (S > 1) {
      gid0 = atomicAdd(&s_groups, tiles);
      rec0 = atomicAdd(&s_recs, tiles * S);
      for (int j = 0; j < tiles; ++j) groups[gid0 + j] = make_int4(b, hf(j), rec0 + j * S, S);
    }
    for (int j = 0; j < tiles; ++j) {
      for (int sp = 0; sp < S; ++sp) {
        const int64_t qpos = (int64_t)pos + j * S + sp;  // < cap_q: cap_q bounds the launch's units
        const int wv = S > 1 ? (gid0 + j) | (sp << 20) | ((S - 1) << 25) : -1;
        if (qpos < cap_q) {
          units[(int64_t)x * cap_q + qpos] = make_int4(b, hf(j), rec0 + j * S, wv);
        }
      }
    }
    carry += __shfl(incl, 63);
  }
  if (lane == 0) s_len[x] = carry;
  __syncthreads();
  if (tid < kXcds) header[kHdrQueueLen + tid] = min(s_len[tid], cap_q);
  if (tid == 0) {
    int total = 0;
    for (int i = 0; i < kXcds; ++i) total += min(s_len[i], cap_q);
    header[kHdrUnits] = total;
    header[kHdrGroups] = s_groups;
    header[kHdrGroupsOff] = groups_off;
    header[kHdrRecordsOff] = records_off;
    header[kHdrRecBytes] = rec_bytes;
    header[kHdrCap] = cap_q;
  }
}

// ---------------------------------------------------------------------------
// Per-workgroup problem description resolved from its work unit.
// ---------------------------------------------------------------------------
struct KvSeg {
  const char* k;
  const char* v;
  int64_t kbase, vbase;  // element offset of key 0, or the head offset when lookup
  int64_t ksn, vsn;      // row strides
  int64_t ksb, vsb;      // sequence strides (lookup only)
  int n;                 // number of keys
  bool lookup;           // keys are packed token indices over a padded tensor
  const int32_t* pages;  // paged segment: page of each FMLM_PAGE_ROWS-key tile, else NULL
  int64_t page_elems;    // elements between pages
  int npool;             // pages in the pool (page ids are clamped to it)
  int ntab;              // entries of the segment's block-table row
};

struct WorkItem {
  int b, h;
  int split_s, split_n;  // part s of S of the key range (S = 1: whole range)
  int split_group, rec0; // split group and its first record
  int qpos0, qcount;     // query positions [qpos0, qpos0+qcount) of sequence b, or with
                         // head-packed tiles rows [qpos0, ...) of its H*len (head, pos) rows
  int len, q0;           // sequence length and packed start (head-packed tiles)
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

// Row statistic for the backward (fmlm_attn_params::lse): log2 of the sum of 2^z over the
// row's keys, from a reference max m and l = sum 2^(z - m); +inf for a row without keys.
// Row pos of sequence b (packed start q0) and head h.
FMLM_DEV void store_lse(const fmlm_attn_params& p, int h, int q0, int pos, float m, float l) {
  p.lse[(int64_t)h * p.total_q + q0 + pos] = l > 0.f ? m + __log2f(l) : INFINITY;
}

FMLM_DEV int4 ldc4(const int4* a, int i) {
  const int32_t* q = (const int32_t*)(a + i);
  return make_int4(ldc(q, 0), ldc(q, 1), ldc(q, 2), ldc(q, 3));
}

// Unit u of a call: packed calls read queue entry u, dense calls map slot u (XCD u % 8,
// position u / 8; group g = (b, h) has its ceil(N/BQ) tiles at consecutive positions of
// XCD g % 8).  Returns false for a unit with nothing to do (an idle dense slot, or an entry
// of a schedule built for other shapes).
FMLM_DEV bool resolve_work(const fmlm_attn_params& p, const int4* units, int u, int BQ, WorkItem& w, bool hpack = false) {
  int b, h, tile;
  w.split_s = 0;
  w.split_n = 1;
  w.split_group = 0;
  w.rec0 = 0;
  w.qcount = 0;
  if (p.cu_seqlens_q) {
    const int4 un = ldc4(units, u);
    b = un.x;
    h = un.y & 0xffff;
    tile = (int)((uint32_t)un.y >> 16);
    if (b < 0 || b >= p.B || h >= p.H) return false;
    if (un.w >= 0) {
      w.split_group = un.w & 0xfffff;
      w.split_s = (un.w >> 20) & 31;
      w.split_n = ((un.w >> 25) & 15) + 1;
      w.rec0 = un.z;
    }
  } else {
    const int nt = (p.N + BQ - 1) / BQ;
    const int x = u % kXcds, pos = u / kXcds;
    const int g = (pos / nt) * kXcds + x;
    tile = pos % nt;
    if (g >= p.B * p.H) return false;
    b = g / p.H;
    h = g - b * p.H;
  }
  const int32_t* cu = p.cu_seqlens_q;
  const SeqInfo si = seq_info(p, b);
  const int q0 = si.q0;
  const int L = si.len;
  w.b = b;
  w.h = h;
  w.len = L;
  w.q0 = q0;
  w.qpos0 = tile * BQ;
  w.qcount = min(BQ, (hpack ? p.H : 1) * L - w.qpos0);
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
  c.pages = nullptr;
  c.page_elems = 0;
  c.npool = 0;
  c.ntab = 0;
  if (!(p.flags & FMLM_FLAG_PREFILL)) {
    const int cb = ctx_batch_of(p, b);
    int c0, c1;
    ctx_range(p, cb, c0, c1);
    c.n = max(c1 - c0, 0);
    if (p.ctx_block_table) {  // paged: rows come from the batch's pages
      c.pages = p.ctx_block_table + (int64_t)cb * p.ctx_pages_per_batch;
      c.page_elems = p.ctx_page_stride;
      c.npool = p.ctx_rows;
      c.ntab = p.ctx_pages_per_batch;
    }
    c.kbase = p.ctx_block_table ? (int64_t)h * p.c_sh
                                : (int64_t)cb * p.c_sb + (int64_t)h * p.c_sh + (int64_t)c0 * p.c_sn;
    c.vbase = c.kbase;
    c.ksn = c.vsn = p.c_sn;
    c.ksb = c.vsb = 0;
  }
  // main segment (mlm_kernel_impl.py:288-293, 360-379)
  KvSeg& m = w.seg[1];
  m.pages = nullptr;
  m.page_elems = 0;
  m.npool = 0;
  m.ntab = 0;
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
  return true;
}


// ---------------------------------------------------------------------------
// The unit of a workgroup (one unit per workgroup): dense calls map workgroup w to slot w
// of the arithmetic layout; packed calls take queue entries (see the schedule comment
// above).
// ---------------------------------------------------------------------------
// workgroups w < G with w % 8 == q: their static units are entries [0, G_q) of queue q
FMLM_DEV int queue_static(int G, int q) { return (G - q + kXcds - 1) / kXcds; }

// entry w / 8 of queue w % 8, or -1 past the queue's end (the unit of workgroup w of a
// launch over 8 * cap workgroups, where every entry is some workgroup's)
FMLM_DEV int queue_first(const int32_t* hdr, int w) {
  const int x = w % kXcds, j = w / kXcds;
  return j < ldc(hdr, kHdrQueueLen + x) ? x * ldc(hdr, kHdrCap) + j : -1;
}

// The unit of workgroup w of a packed launch over G workgroups, G at least the schedule's
// units: its static entry w / 8 of queue w % 8 when the queue has one, else (a spare)
// the overflow entry (an entry past G_q of some queue q) whose rank in queue order equals
// the spare's rank in workgroup order, or -1.  Spares number sum_q (G_q - min(len_q,
// G_q)), at least the overflow entries' sum_q max(len_q - G_q, 0) since sum_q G_q = G >=
// sum_q len_q, so every entry is some workgroup's.  Uniform scalar arithmetic on the
// eight queue lengths: no atomics, nothing carried between launches.
FMLM_DEV int workgroup_unit(const int32_t* hdr) {
  const int G = gridDim.x, w = blockIdx.x, x = w % kXcds, j0 = w / kXcds;
  const int cap = ldc(hdr, kHdrCap);
  if (j0 < ldc(hdr, kHdrQueueLen + x)) return x * cap + j0;
  // spares before w: queue q's spare positions j < j0 (j <= j0 for q < x)
  int r = 0;
  for (int q = 0; q < kXcds; ++q) {
    const int gq = queue_static(G, q);
    r += max(0, min(gq, j0 + (q < x ? 1 : 0)) - min(ldc(hdr, kHdrQueueLen + q), gq));
  }
  for (int q = 0; q < kXcds; ++q) {
    const int gq = queue_static(G, q), ov = max(0, ldc(hdr, kHdrQueueLen + q) - gq);
    if (r < ov) return q * cap + gq + r;
    r -= ov;
  }
  return -1;
}


// ---------------------------------------------------------------------------
// MFMA kernel (bf16 / fp16)
// ---------------------------------------------------------------------------

template <typename T, int D, int QB, int NW, int BK>
struct MfmaCfg {
  static constexpr int NT = NW * 64;
  static constexpr int BQ = NW * QB * 16;
  static constexpr int KS = D + 8;    // LDS K row stride: 16 rows of a b128 read hit distinct banks
  static constexpr int VS = D + 16;   // LDS V row stride: 8 rows of a tr16 read hit distinct banks
  static constexpr int KTILE = BK * KS;
  static constexpr int VTILE = BK * VS;
  static constexpr int STAGE = KTILE + VTILE;          // elements per pipeline stage
  static constexpr int LDS_BYTES = 2 * STAGE * 2;      // two stages
  static constexpr int KC = (D + 31) / 32;   // 32-wide contraction steps over D
  static constexpr int NDB = D / 16;         // 16-wide output column blocks
  static constexpr int NKB = BK / 16;        // 16-key S^T blocks per tile
  static constexpr int NKS = BK / 32;        // 32-key P.V steps per tile
  static constexpr int C8 = D / 8;           // 16-byte chunks per row
  static constexpr int CHUNKS = BK * C8;     // 16-byte chunks per K (or V) tile
  static constexpr int LPT = (CHUNKS + NT - 1) / NT;  // chunks per thread per tensor
  static_assert(D % 16 == 0 && D >= 16, "head dim");
  static_assert(BK % 32 == 0, "key tile");
};

// Lazy rescaling: the running max used for exp2 only moves when a new row max
// exceeds it by more than this (log2 units), so P <= 2^kRescaleSlack and most tiles
// skip the O / l rescale.  Exact after the final O / l.
constexpr float kRescaleSlack = 8.0f;

template <typename T, int D, int QB, int NW, int BK>
__global__ __launch_bounds__(NW * 64, NW >= 8 ? 1 : 2) void attn_mfma_kernel(const fmlm_attn_params p,
                                                               const int4* __restrict__ units,
                                                               const int32_t* __restrict__ hdr) {
  typedef MfmaCfg<T, D, QB, NW, BK> C;
  typedef typename Mfma<T>::v8 v8;
  extern __shared__ __align__(16) char smem_raw[];
  T* const lds = (T*)smem_raw;

  const int u = p.cu_seqlens_q ? workgroup_unit(hdr) : (int)blockIdx.x;
  WorkItem w;
  if (u < 0 || !resolve_work(p, units, u, C::BQ, w)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int32_t* cu = p.cu_seqlens_q;
  const int B = p.B;
  // softmax(scale * s): a negative scale is folded into Q's sign so the exponent
  // scale c is positive; a tiny floor keeps -inf * c == -inf for masked keys.
  const uint32_t qsign = p.scale < 0.f ? 0x80008000u : 0u;
  const float c = fmaxf(fabsf(p.scale) * kLog2e, 1e-30f);

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
      u32x4 raw = u32x4{0u, 0u, 0u, 0u};
      if (ok && col < D) raw = *(const u32x4*)(qbase + (off + col) * 2);
      raw ^= qsign;
      qf[qb][kc] = __builtin_bit_cast(v8, raw);
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

  // ---- tile sequence: context tiles then main tiles
  const int nt0 = (w.seg[0].n + BK - 1) / BK;
  const int nt1 = (w.seg[1].n + BK - 1) / BK;
  const int ntiles = nt0 + nt1;

  // global -> register prefetch of one K and one V tile (16-byte chunks, row-major)
  u32x4 kreg[C::LPT], vreg[C::LPT];
  auto issue_loads = [&](int t) {
    const KvSeg& s = t < nt0 ? w.seg[0] : w.seg[1];
    const int j0 = (t < nt0 ? t : t - nt0) * BK;
    if (!s.lookup) {
      // tile base is workgroup-uniform; each chunk adds a 32-bit element offset
      const char* kt = s.k + (s.kbase + (int64_t)j0 * s.ksn) * 2;
      const char* vt = s.v + (s.vbase + (int64_t)j0 * s.vsn) * 2;
      const int ksn = (int)s.ksn, vsn = (int)s.vsn;
      const bool full = j0 + BK <= s.n;
#pragma unroll
      for (int li = 0; li < C::LPT; ++li) {
        const int it = tid + li * C::NT;
        const int row = it / C::C8, c8 = it % C::C8;
        const bool ok = (C::CHUNKS % C::NT == 0 || it < C::CHUNKS) && (full || j0 + row < s.n);
        kreg[li] = u32x4{0u, 0u, 0u, 0u};
        vreg[li] = u32x4{0u, 0u, 0u, 0u};
        if (ok) {
          kreg[li] = *(const u32x4*)(kt + (int64_t)(row * ksn + c8 * 8) * 2);
          vreg[li] = *(const u32x4*)(vt + (int64_t)(row * vsn + c8 * 8) * 2);
        }
      }
      return;
    }
#pragma unroll
    for (int li = 0; li < C::LPT; ++li) {
      const int it = tid + li * C::NT;
      const int row = it / C::C8, c8 = it % C::C8;
      const int key = j0 + row;
      kreg[li] = u32x4{0u, 0u, 0u, 0u};
      vreg[li] = u32x4{0u, 0u, 0u, 0u};
      if ((C::CHUNKS % C::NT == 0 || it < C::CHUNKS) && key < s.n) {
        const int64_t kr = seg_row(s, key, false, cu, B);
        const int64_t vr = seg_row(s, key, true, cu, B);
        kreg[li] = *(const u32x4*)(s.k + (kr + c8 * 8) * 2);
        vreg[li] = *(const u32x4*)(s.v + (vr + c8 * 8) * 2);
      }
    }
  };
  auto store_lds = [&](int stage) {
    T* Ks = lds + stage * C::STAGE;
    T* Vs = Ks + C::KTILE;
#pragma unroll
    for (int li = 0; li < C::LPT; ++li) {
      const int it = tid + li * C::NT;
      if (C::CHUNKS % C::NT != 0 && it >= C::CHUNKS) continue;
      const int row = it / C::C8, c8 = it % C::C8;
      *(u32x4*)(Ks + row * C::KS + c8 * 8) = kreg[li];
      *(u32x4*)(Vs + row * C::VS + c8 * 8) = vreg[li];
    }
  };

  if (ntiles > 0) {
    issue_loads(0);
    store_lds(0);
    if (ntiles > 1) issue_loads(1);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int stage = t & 1;
    const T* Ks = lds + stage * C::STAGE;
    const T* Vs = Ks + C::KTILE;
    const int nk = t < nt0 ? min(BK, w.seg[0].n - t * BK) : min(BK, w.seg[1].n - (t - nt0) * BK);

    // ---- S^T = K Q^T: accumulator lane (q + 16g) reg r = S[query q][key 16kb + 4g + r]
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

    // the other stage is free: land the prefetched tile there and fetch the next
    if (t + 1 < ntiles) {
      store_lds(stage ^ 1);
      if (t + 2 < ntiles) issue_loads(t + 2);
    }

    // ---- online softmax (mlm_kernel_impl.py:42-60); lane owns query l16 of each block
    if (nk < BK) {
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kb * 16 + g * 4 + r >= nk)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) s[kb][qb][r] = -INFINITY;
    }
    v8 pf[C::NKS][QB];
    bool need_rescale = false;
    float m_new[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = s[0][qb][0];
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
        for (int r = (kb == 0 ? 1 : 0); r < 4; ++r) mx = fmaxf(mx, s[kb][qb][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      mx *= c;
      const bool grow = mx > m_i[qb] + kRescaleSlack;
      m_new[qb] = grow ? mx : m_i[qb];
      need_rescale = need_rescale || grow;
    }
    if (__builtin_amdgcn_ballot_w64(need_rescale)) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const float alpha = fast_exp2(m_i[qb] - m_new[qb]);  // 1 where unchanged, 0 on the first tile
        m_i[qb] = m_new[qb];
        l_i[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) o[db][qb] *= alpha;
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float mneg = -m_i[qb];
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = fast_exp2(fmaf(s[kb][qb][r], c, mneg));
          rs += pv;
          pf[kb >> 1][qb][(kb & 1) * 4 + r] = (T)pv;
        }
      }
      l_i[qb] += rs;
    }

    // ---- O^T += V^T P^T; the V^T fragment comes from row-major V via two tr16 reads:
    // lane (j + 16g) addresses V[32ks + 16h + 4g + j/4][16db + 4(j%4)], h = 0, 1, so lane
    // (i + 16g) receives V[32ks + 16h + 4g + e][16db + i] -- the keys of its P^T elements.
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        const T* base = Vs + (ks * 32 + g * 4 + (l16 >> 2)) * C::VS + db * 16 + (l16 & 3) * 4;
        const s16x4 lo = lds_read_tr16(base);
        const s16x4 hi = lds_read_tr16(base + 16 * C::VS);
        const v8 a = __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[db][qb] = Mfma<T>::run(a, pf[ks][qb], o[db][qb]);
      }
    }
    __syncthreads();  // this stage is consumed; the next one is complete
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
    if (p.lse && g == 0) store_lse(p, w.h, w.q0, w.qpos0 + row, m_i[qb], l);
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
// Software-pipelined MFMA kernel (v3) for head dims 16..256.
//
// The LDS holds two K tiles and three V tiles, filled by direct global->LDS loads (no
// staging registers) with 16-byte chunks XOR-swizzled per row (K tiles by k_swz, V tiles
// by kv_swz), so both the b128 K reads and the tr16 V reads are bank-conflict free.
// Iteration t of a wave:
//   1. issues the loads of K(t+2) (into K(t)'s buffer) and V(t+2) (into V(t-1)'s);
//   2. row max of S(t) (lane-local + two permlane swaps) and the lazy-rescale decision;
//   3. one basic block that runs S(t+1) = K(t+1) Q^T on the MFMA pipe while the VALU
//      computes P(t) = exp2(S(t) c - m), then O += V(t)^T P(t) and l += 1^T P(t) (the row
//      sums as an MFMA against a ones operand);
//   4. waits for its loads except V(t+2)'s, which have until the end of step t+1 (every
//      wave issues the same number of loads per tile, so vmcnt leaves exactly those in
//      flight), and meets the other waves at a barrier.
// The loads are issued with inline asm: the compiler cannot tell the LDS writes of a
// global_load_lds builtin from the V reads of the same iteration and would otherwise
// wait for every outstanding load before the first V read; ordering is enforced here
// by the explicit wait + barrier of step 4 instead.
// ---------------------------------------------------------------------------

// Page ids of 64 consecutive key tiles of a paged segment, one per lane of a VGPR: a tile
// then costs a lane read.  A page id fetched per tile by a vector load would make its use
// wait for every outstanding vector memory operation, the in-flight tile loads too; the
// window's reload pays that wait once per 64 tiles.
struct PageWindow {
  int ids;    // lane i: page of tile first + i
  int first;  // first tile of the window
};
FMLM_DEV void page_window_reset(PageWindow& w) { w.first = -(1 << 30); }
// byte offset of tile `tile`'s page from the paged segment's page 0 (page ids clamped to
// the pool)
FMLM_DEV int64_t page_offset(const KvSeg& s, int tile, PageWindow& w) {
  tile = __builtin_amdgcn_readfirstlane(tile);
  if ((unsigned)(tile - w.first) >= 64u) {
    w.first = tile;
    const int lane = threadIdx.x & 63;
    w.ids = s.pages[min(tile + lane, max(s.ntab - 1, 0))];
    // consume the load here: the wait for it then stays on this path, not after the join
    asm volatile("" ::"v"(w.ids));
  }
  int pg = __builtin_amdgcn_readlane(w.ids, tile - w.first);
  pg = min(max(pg, 0), max(s.npool - 1, 0));
  return (int64_t)pg * s.page_elems * 2;
}
// first row of tile `tile` of a paged segment
FMLM_DEV const char* page_row0(const KvSeg& s, const char* base, int tile, PageWindow& w) {
  return base + page_offset(s, tile, w);
}

// walks the key tiles of a work item for the direct loads (see attn_mfma3_kernel)
struct KeyCursor {
  const char* p;     // row 0 of the current tile
  const char* base;  // the segment's first row (paged: its row 0 of page 0 of the pool)
  uint32_t rowb;
  int left, seg, tile;
  PageWindow pw;     // paged segment: page ids of the tiles around `tile`
};

// the single-group schedule's walk: K and V of a key tile are loaded together, so one
// position (segment, keys left, tile, page) serves both tensors
struct PairCursor {
  const char* pk;  // row 0 of the next K / V tile to load
  const char* pv;
  const char* bk;  // the segment's first K / V row (paged: row 0 of page 0 of the pool)
  const char* bv;
  int64_t stk, stv;     // bytes from one tile's row 0 to the next's
  uint32_t rowk, rowv;  // row pitches in bytes
  int ft;               // the next tile to load (index over both segments)
  bool full_pitch;  // both pitches equal the main K pitch of the precomputed lane offsets
  PageWindow pw;
};

// PPB > 0: the ping-pong schedule (8 waves in two groups of 4, one half-step apart) with
// PPB buffers per tensor; 0: the single-group schedule with K[2], V[3]
template <typename T, int D, int QB, int NW, int BK, int PPB = 0>
struct Mfma3Cfg {
  static constexpr bool PP = PPB > 0;
  static constexpr int NT = NW * 64;
  static constexpr int BQ = NW * QB * 16;
  static constexpr int ROWB = D * 2;          // bytes per K / V row (unpadded)
  static constexpr int TILEB = BK * ROWB;
  static constexpr int CPR = D / 8;           // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;        // rows per wave-wide direct load
  static constexpr int NINST = BK / RPI;      // wave-wide loads per tile per tensor
  static constexpr int NPW = (NINST + NW - 1) / NW;  // ... per wave
  static constexpr int NKBUF = PP ? PPB : 2;
  static constexpr int NVBUF = PP ? PPB : 3;
  static constexpr int LDS_BYTES = (NKBUF + NVBUF) * TILEB;
  static constexpr int KC = (D + 31) / 32;
  static constexpr int NDB = D / 16;
  static constexpr int NKB = BK / 16;
  static constexpr int NKS = BK / 32;
  static constexpr int LEAD = D <= 64 ? 2 : 3;  // LDS fragment reads in flight ahead of use
  static constexpr int NKF = KC * NKB;    // K fragment reads per step
  static constexpr int NVF = NKS * NDB;   // V fragment (tr16 pair) reads per step
  static_assert(D % 16 == 0 && D >= 16 && D <= 256, "head dim");
  static_assert(BK % 32 == 0 && BK % RPI == 0, "key tile");
  static_assert(!PP || (NW == 8 && NINST % NW == 0 && PPB >= 3), "ping-pong: two groups of 4 waves, equal loads");
};

template <typename T, int D, int QB, int NW, int BK, bool PAGED, int PPB>
__global__ __launch_bounds__(NW * 64, NW >= 8 ? 1 : 2) void attn_mfma3_kernel(
    const fmlm_attn_params p, const int4* __restrict__ units, const int32_t* __restrict__ hdr) {
  typedef Mfma3Cfg<T, D, QB, NW, BK, PPB> C;
  typedef typename Mfma<T>::v8 v8;
  extern __shared__ __align__(16) char smem_raw[];
  char* const kbuf = smem_raw;                             // [NKBUF][TILEB]
  char* const vbuf = smem_raw + C::NKBUF * C::TILEB;       // [NVBUF][TILEB]

  const int u = p.cu_seqlens_q ? workgroup_unit(hdr) : (int)blockIdx.x;
  WorkItem w;
  if (u < 0 || !resolve_work(p, units, u, C::BQ, w)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15;
  const int g = lane >> 4;
  // ---- Q fragments (B operand of S^T): lane (q + 16g), block qb, step kc.  fp16: pre-scaled
  // by scale*log2(e) (one rounding to the input type) so that S comes out of the MFMAs in
  // log2 units.  bf16 (FP32_SCALE): as stored but for the sign of a negative scale, with
  // c = |scale|*log2(e) applied in fp32 to the accumulators (the running max kept in log2
  // units, the accumulators' in raw units): bf16's 8-bit mantissa would round q*c to an
  // error that large scores turn into a tilt of P past the output tolerance, as the
  // reference's fp32-scaled product does not; fp16's 11 bits keep it below.  The floor
  // keeps -inf * c == -inf for masked keys at scale 0.
  constexpr bool FP32_SCALE = std::is_same<T, bf16>::value;
  const float cs = p.scale * kLog2e;
  const uint32_t qsign = p.scale < 0.f ? 0x80008000u : 0u;
  const float c = fmaxf(fabsf(p.scale) * kLog2e, 1e-30f);
  const float rc = 1.f / c;
  v8 qf[QB][C::KC];
  auto load_q = [&]() {
    const char* qbase = (const char*)p.q;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int row = (wave * QB + qb) * 16 + l16;
      const bool ok = row < w.qcount;
      const int64_t off = w.q_row0 + (int64_t)row * w.q_sn;
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc) {
        const int col = kc * 32 + g * 8;
        if constexpr (FP32_SCALE) {
          u32x4 raw = u32x4{0u, 0u, 0u, 0u};
          if (ok && col < D) raw = *(const u32x4*)(qbase + (off + col) * 2);
          qf[qb][kc] = __builtin_bit_cast(v8, raw ^ qsign);
        } else {
          v8 raw = v8{};
          if (ok && col < D) raw = *(const v8*)(qbase + (off + col) * 2);
#pragma unroll
          for (int e = 0; e < 8; ++e) raw[e] = (T)((float)raw[e] * cs);
          qf[qb][kc] = raw;
        }
      }
    }
  };
  if constexpr (C::PP) load_q();  // the single-group schedule loads Q after its first tiles

  // ---- per-lane LDS byte addresses (see k_swz / kv_swz): the K fragment of block kb,
  // step kc of the K tile at byte offset o from the first K buffer is at koff[kc%4] + o +
  // kb*16*ROWB + 256*(kc/4); the V tr16 fragment of step ks, column block db, half h of
  // the V tile at offset o from the first V buffer at voff[db%8] + o + (32 ks + 16 h)*ROWB
  // + 256*(db/8).  The lane's register then carries the whole address and every other
  // term is a read's immediate offset (a constant in the unrolled steps).
  uint32_t koff[4], voff[8];
  {
    const int ksw = k_swz<D>(l16);
#pragma unroll
    for (int b = 0; b < 4; ++b) koff[b] = lds_addr(kbuf) + l16 * C::ROWB + 16 * ((4 * b + g) ^ ksw);
    const int vr = 4 * g + (l16 >> 2);
    const int vsw = kv_swz<D>(vr);
    const int x = (l16 & 3) >> 1;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      voff[db] = lds_addr(vbuf) + vr * C::ROWB + 16 * ((2 * db + x) ^ vsw) + 8 * (l16 & 1);
  }
  // ---- per-lane direct-load layout: wave-wide load i = wave + j*NW brings rows
  // [i*RPI, (i+1)*RPI); lane l fetches logical chunk (l % CPR) ^ swz(row) of row
  // i*RPI + l/CPR, which lands in physical chunk l % CPR (swz: k_swz for K tiles, read by
  // b128 only; kv_swz for V tiles, read by tr16 only)
  const int drow0 = wave * C::RPI + lane / C::CPR;  // + j*NW*RPI for load j

  f32x4 o[C::NDB][QB];
  f32x4 lsum[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    lsum[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // m_i: running row maximum (log2 units); sbase: the maximum the current S tile was
  // computed against (its accumulators start at -sb)
  float m_i[QB], sbase[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = -INFINITY;
    sbase[qb] = 0.f;
  }
  const bool wave_active = wave * QB * 16 < w.qcount;
  KeyCursor kcur, vcur;  // ping-pong schedule
  PairCursor pc;         // single-group schedule
  // LDS byte addresses of the buffers, kept in registers (the empty asm stops the compiler
  // from recomputing them from the shared aperture at every use)
  uint32_t kl = lds_addr(kbuf), vl = lds_addr(vbuf);
  asm volatile("" : "+s"(kl), "+s"(vl));

  const int nt0 = (w.seg[0].n + BK - 1) / BK;
  const int nt1 = (w.seg[1].n + BK - 1) / BK;
  const int ntiles = nt0 + nt1;
  // key tiles [tb, te) of this unit: all of them, or part s of S of a split group
  const int tb = (int)((int64_t)w.split_s * ntiles / w.split_n);
  const int te = (int)((int64_t)(w.split_s + 1) * ntiles / w.split_n);
  // the partial last tile of each segment (-1: none) and the keys it holds; every other
  // tile holds BK keys
  const int pt0 = (w.seg[0].n % BK) ? nt0 - 1 : -1, pt1 = (w.seg[1].n % BK) ? ntiles - 1 : -1;
  const int nk0 = w.seg[0].n - (nt0 - 1) * BK, nk1 = w.seg[1].n - (nt1 - 1) * BK;

  // ---- direct loads.  A cursor walks the key tiles of the context then the main segment
  // (linear addressing: the dispatcher routes per-row lookups elsewhere): p is the
  // wave-uniform byte address of the current tile's row 0, left the keys left in the
  // segment from there.  Rows past a segment end repeat its last row (their scores are
  // masked to -inf, so P = 0 multiplies finite values).
  typedef KeyCursor Cursor;
  auto lane_offsets = [&](uint32_t rowb, int last, bool is_v, uint32_t (&ofs)[C::NPW]) {
#pragma unroll
    for (int j = 0; j < C::NPW; ++j) {
      const int row = drow0 + j * NW * C::RPI;
      const int sw = is_v ? kv_swz<D>(row) : k_swz<D>(row);
      ofs[j] = (uint32_t)__umul24((uint32_t)min(row, last), rowb) + 16 * ((lane % C::CPR) ^ sw);
    }
  };
  // a paged context (PAGED instantiation, segment 0 only) puts each key tile in a page
  const bool ctx_paged = PAGED && w.seg[0].pages != nullptr;
  auto cursor_seg = [&](Cursor& cr, int sg, bool is_v) {
    const KvSeg& sgm = w.seg[sg];
    cr.seg = sg;
    cr.tile = 0;
    cr.left = __builtin_amdgcn_readfirstlane(sgm.n);
    cr.rowb = __builtin_amdgcn_readfirstlane((uint32_t)(is_v ? sgm.vsn : sgm.ksn) * 2u);
    cr.base = uniform_ptr((is_v ? sgm.v : sgm.k) + (is_v ? sgm.vbase : sgm.kbase) * 2);
    cr.p = cr.base;
    page_window_reset(cr.pw);
    if constexpr (PAGED)
      if (sg == 0 && ctx_paged && cr.left > 0) cr.p = uniform_ptr(page_row0(w.seg[0], cr.base, 0, cr.pw));
  };
  // position a cursor on key tile t
  auto cursor_seek = [&](Cursor& cr, int t, bool is_v) {
    const int sg = t < nt0 ? 0 : 1;
    cursor_seg(cr, sg, is_v);
    const int skip = sg == 0 ? t : t - nt0;
    cr.left -= skip * BK;
    cr.tile = skip;
    if (PAGED && sg == 0 && ctx_paged) {
      if constexpr (PAGED) cr.p = cr.left > 0 ? uniform_ptr(page_row0(w.seg[0], cr.base, skip, cr.pw)) : cr.base;
    } else {
      cr.p += (size_t)skip * BK * cr.rowb;
    }
  };
  // lane offsets of a whole tile at the main segment's K row pitch (the common case), for
  // K tiles and V tiles (the same when the two swizzles agree)
  const uint32_t oc_rowb = __builtin_amdgcn_readfirstlane((uint32_t)w.seg[1].ksn * 2u);
  uint32_t oc_k[C::NPW], oc_v[C::NPW];
  lane_offsets(oc_rowb, BK, false, oc_k);
  lane_offsets(oc_rowb, BK, true, oc_v);
  // the paired cursor at the start of segment sg / on key tile t
  auto pair_seg = [&](PairCursor& cr, int sg) {
    const KvSeg& sgm = w.seg[sg];
    cr.rowk = __builtin_amdgcn_readfirstlane((uint32_t)sgm.ksn * 2u);
    cr.rowv = __builtin_amdgcn_readfirstlane((uint32_t)sgm.vsn * 2u);
    cr.stk = (int64_t)cr.rowk * BK;
    cr.stv = (int64_t)cr.rowv * BK;
    cr.full_pitch = cr.rowk == oc_rowb && cr.rowv == oc_rowb;
    cr.bk = uniform_ptr(sgm.k + sgm.kbase * 2);
    cr.bv = uniform_ptr(sgm.v + sgm.vbase * 2);
    cr.pk = cr.bk;
    cr.pv = cr.bv;
    page_window_reset(cr.pw);
  };
  // paged context tile t: the page of K and V from one table read
  auto pair_page = [&](PairCursor& cr, int t) {
    if constexpr (PAGED) {
      const int64_t off = page_offset(w.seg[0], t, cr.pw);
      cr.pk = uniform_ptr(cr.bk + off);
      cr.pv = uniform_ptr(cr.bv + off);
    }
  };
  auto pair_seek = [&](PairCursor& cr, int t) {
    const int sg = t < nt0 ? 0 : 1;
    pair_seg(cr, sg);
    cr.ft = t;
    if (PAGED && sg == 0 && ctx_paged) {
      pair_page(cr, t);
    } else {
      const int skip = sg == 0 ? t : t - nt0;
      cr.pk += skip * cr.stk;
      cr.pv += skip * cr.stv;
    }
  };
  // load the cursor's K tile into LDS byte address kdst and its V tile into vdst (K's loads
  // issued first), then advance to the next tile
  auto fetch_pair = [&](PairCursor& cr, uint32_t kdst, uint32_t vdst) {
    const int t = cr.ft;
    const bool part = t == pt0 || t == pt1;
    uint32_t ok[C::NPW], ov[C::NPW];
    if (!part && cr.full_pitch) {
#pragma unroll
      for (int j = 0; j < C::NPW; ++j) {
        ok[j] = oc_k[j];
        ov[j] = oc_v[j];
      }
    } else {
      const int last = !part ? BK - 1 : (t == pt0 ? nk0 : nk1) - 1;
      lane_offsets(cr.rowk, last, false, ok);
      lane_offsets(cr.rowv, last, true, ov);
    }
#pragma unroll
    for (int j = 0; j < C::NPW; ++j) {
      const int i = wave + j * NW;
      if (C::NINST % NW == 0 || i < C::NINST)
        dma16_sbase(cr.pk, ok[j], __builtin_amdgcn_readfirstlane(kdst + i * 1024));
    }
#pragma unroll
    for (int j = 0; j < C::NPW; ++j) {
      const int i = wave + j * NW;
      if (C::NINST % NW == 0 || i < C::NINST)
        dma16_sbase(cr.pv, ov[j], __builtin_amdgcn_readfirstlane(vdst + i * 1024));
    }
    cr.ft = t + 1;
    if (t + 1 == nt0) {  // the main segment's first tile next
      pair_seg(cr, 1);
    } else if (PAGED && ctx_paged && t + 1 < nt0) {  // one page per context tile
      pair_page(cr, t + 1);
    } else {
      cr.pk += cr.stk;
      cr.pv += cr.stv;
    }
  };
  // load the cursor's tile into LDS dst and advance to the next tile
  auto fetch = [&](Cursor& cr, char* dst, bool is_v) {
    const uint32_t lds0 = lds_addr(dst);
    uint32_t ofs[C::NPW];
    if (cr.left >= BK && cr.rowb == oc_rowb) {
#pragma unroll
      for (int j = 0; j < C::NPW; ++j) ofs[j] = is_v ? oc_v[j] : oc_k[j];
    } else {
      lane_offsets(cr.rowb, cr.left - 1, is_v, ofs);
    }
#pragma unroll
    for (int j = 0; j < C::NPW; ++j) {
      const int i = wave + j * NW;
      if (C::NINST % NW == 0 || i < C::NINST)
        dma16_sbase(uniform_ptr(cr.p), ofs[j], __builtin_amdgcn_readfirstlane(lds0 + i * 1024));
    }
    cr.left -= BK;
    cr.tile += 1;
    if (PAGED && cr.seg == 0 && ctx_paged) {  // one page per context tile
      if constexpr (PAGED) cr.p = cr.left > 0 ? uniform_ptr(page_row0(w.seg[0], cr.base, cr.tile, cr.pw)) : cr.base;
    } else {
      cr.p += (size_t)BK * cr.rowb;
    }
    if (cr.left <= 0 && cr.seg == 0 && w.seg[1].n > 0) cursor_seg(cr, 1, is_v);
  };
  auto tile_keys = [&](int t) { return t == pt0 ? nk0 : t == pt1 ? nk1 : BK; };
  // S^T = K Q^T from the K tile at byte offset kt from the first K buffer (prologue only;
  // the steps interleave it)
  auto qk = [&](uint32_t kt, f32x4 (&s)[C::NKB][QB]) {
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
        v8 a;
        if (kc * 32 + g * 8 < D)
          a = *(const FMLM_LDS v8*)(uintptr_t)(koff[kc & 3] + kt + kb * 16 * C::ROWB + 256 * (kc >> 2));
        else
          a = v8{};
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          s[kb][qb] = Mfma<T>::run(a, qf[qb][kc], kc == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[kb][qb]);
      }
    }
  };
  v8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (T)1.0f;
  pin(ones);  // keep in registers rather than rematerialised per use

  // raw row maxima of a score tile (before the scale); rows past a segment end repeat
  // its last valid row, so they never change a maximum
  auto row_max = [&](const f32x4 (&sx)[C::NKB][QB], float (&mx)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float m = vmax(vmax(sx[0][qb][0], sx[0][qb][1]), vmax(sx[0][qb][2], sx[0][qb][3]));
#pragma unroll
      for (int kb = 1; kb < C::NKB; ++kb)
        m = vmax(vmax(m, vmax(sx[kb][qb][0], sx[kb][qb][1])), vmax(sx[kb][qb][2], sx[kb][qb][3]));
      mx[qb] = lane_max_xor16_32(m);
    }
  };

  // end of step t: wait for every load but V(t+2)'s (needed only at step t+2; loads
  // complete in issue order, and they were issued last).  When the waves issue unequal
  // numbers of loads (tiny tiles), wait for all.
  auto vwait = [&](int t) {
    constexpr int VPW = C::NINST / NW;
    if (C::NINST % NW == 0 && t + 2 < te)
      __builtin_amdgcn_s_waitcnt((VPW & 15) | (7 << 4) | (15 << 8) | ((VPW >> 4) << 14));
    else
      __builtin_amdgcn_s_waitcnt(0);
  };
  // Rescale decision for tile t from the row maxima mx of S(t) (sc), and the -inf mask of
  // the keys past a partial tile's end.
  auto prepare = [&](int t, f32x4 (&sc)[C::NKB][QB], float (&mx)[QB]) {
    bool need_rescale = false;
    float m_new[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float m = FP32_SCALE ? fmaf(mx[qb], c, sbase[qb]) : mx[qb] + sbase[qb];
      const bool grow = m > m_i[qb] + kRescaleSlack;
      m_new[qb] = grow ? m : m_i[qb];
      need_rescale = need_rescale || grow;
    }
    if (__builtin_amdgcn_ballot_w64(need_rescale)) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const float alpha = fast_exp2(m_i[qb] - m_new[qb]);  // 1 where unchanged, 0 on the first tile
        const float shift = FP32_SCALE ? (sbase[qb] - m_new[qb]) * rc : sbase[qb] - m_new[qb];  // 0 where unchanged
        m_i[qb] = m_new[qb];
        lsum[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) o[db][qb] *= alpha;
#pragma unroll
        for (int kb = 0; kb < C::NKB; ++kb) sc[kb][qb] += shift;
      }
    }
    const int nk = tile_keys(t);
    if (nk < BK) {
      const int lim = nk - 4 * g;  // key kb*16 + 4g + r is valid iff kb*16 + r < lim
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kb * 16 + r >= lim)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) sc[kb][qb][r] = -INFINITY;
    }
  };

  // ---- the fused block of a step, as a sequence of slots fenced by sched_barrier so the
  // order below is the issue order.  Slot s runs the MFMAs of operand fragment s:
  // fragments [0, NKF) are K(t+1) fragments (S(t+1) = sn from the K tile at byte offset kn
  // from the first K buffer, beside a share of the exp work of P(t) from sc), fragments
  // [NKF, NKF+NVF) are V(t) fragments (O += V^T P from the V tile at byte offset vt from
  // the first V buffer, beside a share of the row-max work of S(t+1) into mx).  The LDS
  // read of fragment s + C::LEAD is issued at the top of slot s (within [S0, S1)).  Phase A
  // (slots [0, NKF)) leaves P(t) in pf for phase B.
  constexpr int NF = C::NKF + C::NVF;
  constexpr int NP = C::NKB * QB * 2;    // exp pairs
  constexpr int NMS = C::NKB * QB + QB;  // row-max steps
  u32x4 pf[C::NKS][QB];  // P(t) as packed pairs, the B operand of P V
  float mpart[QB], mhold[QB];
  auto run_slots = [&](auto s0c, auto s1c, f32x4 (&sc)[C::NKB][QB], f32x4 (&sn)[C::NKB][QB],
                       float (&mx)[QB], uint32_t kn, uint32_t vt) {
    constexpr int S0 = decltype(s0c)::value, S1 = decltype(s1c)::value;
    f32x4 minit[QB];  // -m_i splat (in the accumulators' units): the initial S accumulators
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float mr = FP32_SCALE ? -m_i[qb] * rc : -m_i[qb];
      minit[qb] = f32x4{mr, mr, mr, mr};
    }
    v8 fr[C::LEAD + 1];
    auto issue = [&](int r) {
      if (r < C::NKF) {
        const int kc = r / C::NKB, kb = r % C::NKB;
        fr[r % (C::LEAD + 1)] = kc * 32 + g * 8 < D
            ? *(const FMLM_LDS v8*)(uintptr_t)(koff[kc & 3] + kn + kb * 16 * C::ROWB + 256 * (kc >> 2)) : v8{};
      } else {
        const int j = r - C::NKF, ks = j / C::NDB, db = j % C::NDB;
        const uint32_t va = voff[db & 7] + vt + ks * 32 * C::ROWB + 256 * (db >> 3);
        const s16x4 lo = lds_read_tr16_at(va);
        const s16x4 hi = lds_read_tr16_at(va + 16 * C::ROWB);
        fr[r % (C::LEAD + 1)] = __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    // exp of S^T elements (kb, r), (kb, r+1) of block qb; keys kb*16 + 4g + r (+1) are
    // elements (kb&1)*4 + r (+1) of the P fragment of key step kb/2.  pin() keeps the
    // work inside its slot (pure arithmetic would otherwise be moved to its first use).
    auto exp_pair = [&](int pi) {
      const int qb = pi / (C::NKB * 2), kb = (pi >> 1) % C::NKB, r = (pi & 1) * 2;
      if (r == 0) pin(sc[kb][qb]);
      f32x2 x = f32x2{sc[kb][qb][r], sc[kb][qb][r + 1]};
      x[0] = fast_exp2(FP32_SCALE ? x[0] * c : x[0]);
      x[1] = fast_exp2(FP32_SCALE ? x[1] * c : x[1]);
      uint32_t wv = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, typename Pair<T>::type));
      pin(wv);
      pf[kb >> 1][qb][(kb & 1) * 2 + (pi & 1)] = wv;
    };
    auto max_step = [&](int k) {
      if (k < C::NKB * QB) {
        const int qb = k / C::NKB, kb = k % C::NKB;
        pin(sn[kb][qb]);
        const f32x4 x = sn[kb][qb];
        // one running max3 chain over the 4 * NKB values of the row block, a value held
        // back per block so that every step folds two new values (8 ops at NKB = 4)
        if (kb == 0) {
          mpart[qb] = vmax(vmax(x[0], x[1]), x[2]);
        } else {
          mpart[qb] = vmax(vmax(mpart[qb], mhold[qb]), x[0]);
          mpart[qb] = vmax(vmax(mpart[qb], x[1]), x[2]);
        }
        mhold[qb] = x[3];
        if (kb == C::NKB - 1) mpart[qb] = vmax(mpart[qb], mhold[qb]);
        pin(mpart[qb]);
      } else {
        const int qb = k - C::NKB * QB;
        mx[qb] = lane_max_xor16_32(mpart[qb]);
        pin(mx[qb]);
      }
    };
#pragma unroll
    for (int r = S0; r < S0 + C::LEAD && r < S1; ++r) issue(r);
    // wave priority: a wave in its MFMA-dense block issues ahead of the other waves on its
    // SIMD (their loads, branches and softmax VALU fill the gaps), the P V phase highest
    __builtin_amdgcn_s_setprio(S0 < C::NKF ? 1 : 2);
#pragma unroll
    for (int sl = S0; sl < S1; ++sl) {
      if (sl + C::LEAD < S1) issue(sl + C::LEAD);
      if (sl == C::NKF && sl != S0) __builtin_amdgcn_s_setprio(2);
      const v8 a = fr[sl % (C::LEAD + 1)];
      if (sl < C::NKF) {
        const int kc = sl / C::NKB, kb = sl % C::NKB;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          sn[kb][qb] = Mfma<T>::run(a, qf[qb][kc], kc == 0 ? minit[qb] : sn[kb][qb]);
#pragma unroll
        for (int pi = sl * NP / C::NKF; pi < (sl + 1) * NP / C::NKF; ++pi) exp_pair(pi);
      } else {
        const int j = sl - C::NKF, ks = j / C::NDB, db = j % C::NDB;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          o[db][qb] = Mfma<T>::run(a, __builtin_bit_cast(v8, pf[ks][qb]), o[db][qb]);
        if (db == C::NDB - 1)
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            lsum[qb] = Mfma<T>::run(ones, __builtin_bit_cast(v8, pf[ks][qb]), lsum[qb]);
#pragma unroll
        for (int k = j * NMS / C::NVF; k < (j + 1) * NMS / C::NVF; ++k) max_step(k);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  typedef std::integral_constant<int, 0> Slot0;
  typedef std::integral_constant<int, C::NKF> SlotB;
  typedef std::integral_constant<int, NF> SlotEnd;

  // One pipeline step (single-group schedule): sc holds S(t) and mx its row maxima;
  // computes sn = S(t+1) from the K tile at byte offset kn and its maxima, consumes V(t) at
  // byte offset vt, refills kdst with K(t+2) and vdst with V(t+2).
  auto step = [&](int t, f32x4 (&sc)[C::NKB][QB], f32x4 (&sn)[C::NKB][QB], float (&mx)[QB],
                  uint32_t kn, uint32_t vt, uint32_t kdst, uint32_t vdst) {
    if (t + 2 < te) fetch_pair(pc, kdst, vdst);
    if (!wave_active) {  // every query row of this wave is padding: loads and barriers only
      vwait(t);
      __syncthreads();
      return;
    }
    prepare(t, sc, mx);
    run_slots(Slot0{}, SlotEnd{}, sc, sn, mx, kn, vt);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) sbase[qb] = m_i[qb];
    vwait(t);
    __syncthreads();
  };

  f32x4 sa[C::NKB][QB], sb[C::NKB][QB];
  float mx[QB];
  if constexpr (C::PP) {
    // ---- ping-pong schedule.  Waves w and w + 4 share a SIMD; group gp = w / 4.  A step
    // is two half-steps: A(i) = S(t+1) beside the exp of P(t), B(i) = O += V(t)^T P(t)
    // beside the row maxima of S(t+1) (t = tb + i).  Group 0 runs A(i) in slot 2i and B(i)
    // in slot 2i+1, group 1 one slot later, so in every slot one wave of each SIMD is in
    // its exp-heavy half and the other in its MFMA-dense half.  A barrier ends each slot.
    // Buffers: K(j) in K buffer j % NKBUF, read in slots 2j-2 and 2j-1, refilled (with
    // K(j + NKBUF)) in slot 2j; V(j) in V buffer j % NVBUF, read in slots 2j+1 and 2j+2,
    // refilled (with V(j + NVBUF)) in slot 2j+3.  A load issued in slot s is first read
    // in slot s + 2*NBUF - 2, so it may stay in flight over 2*NBUF - 3 slot ends.
    static_assert(C::NKBUF == C::NVBUF, "one load window for both tensors");
    constexpr int WIN = 2 * C::NKBUF - 3;  // slots whose loads may be in flight at a slot end
    const int gp = wave >> 2;
    const int n = te - tb;
    if (n > 0) {
      cursor_seek(kcur, tb, false);
      cursor_seek(vcur, tb, true);
#pragma unroll
      for (int j = 0; j < C::NKBUF; ++j)
        if (j < n) fetch(kcur, kbuf + j * C::TILEB, false);
#pragma unroll
      for (int j = 0; j < C::NVBUF; ++j)
        if (j < n) fetch(vcur, vbuf + j * C::TILEB, true);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (wave_active) {
        qk(0, sa);
        row_max(sa, mx);
      }
      __syncthreads();  // every wave is done with K(0): its buffer may be refilled
    }
    // the loads of slot s (every wave issues its share of the tile); returns whether any
    int hist = 0;  // bit k: slot s - k issued loads
    auto slot_loads = [&](int s) {
      const int i = s >> 1;
      bool any = false;
      if ((s & 1) == 0) {
        if (i + C::NKBUF < n) {
          fetch(kcur, kbuf + (i % C::NKBUF) * C::TILEB, false);
          any = true;
        }
      } else if (i >= 1 && i - 1 + C::NVBUF < n) {
        fetch(vcur, vbuf + ((i - 1) % C::NVBUF) * C::TILEB, true);
        any = true;
      }
      hist = ((hist << 1) | (any ? 1 : 0)) & ((1 << WIN) - 1);
    };
    // end of a slot: the loads issued before the last WIN slots have landed (all of them
    // unless each of those slots issued its share), then the barrier
    auto slot_end = [&]() {
      if (hist == (1 << WIN) - 1)
        __builtin_amdgcn_s_waitcnt(((WIN * C::NPW) & 15) | (7 << 4) | (15 << 8) | (((WIN * C::NPW) >> 4) << 14));
      else
        __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    };
    auto phase_a = [&](int i, uint32_t kn) {
      if (wave_active) {
        prepare(tb + i, sa, mx);
        run_slots(Slot0{}, SlotB{}, sa, sb, mx, kn, 0u);
      }
    };
    auto phase_b = [&](uint32_t vt) {
      if (wave_active) {
        run_slots(SlotB{}, SlotEnd{}, sa, sb, mx, 0u, vt);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sbase[qb] = m_i[qb];
      }
      // unconditional, so that S(t) is dead after phase A on every path
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sa[kb][qb] = sb[kb][qb];
    };
    if (n > 0) {
      if (gp == 1) {  // group 1 starts one slot late
        slot_loads(0);
        slot_end();
      }
      // step i of the unit: A(i) reads K buffer (i + 1) % NKBUF, B(i) V buffer i % NVBUF;
      // NKBUF steps per iteration make both offsets constants of the unrolled step
      auto pp_step = [&](int i, int u) {
        slot_loads(2 * i + gp);
        phase_a(i, ((u + 1) % C::NKBUF) * C::TILEB);
        slot_end();
        slot_loads(2 * i + 1 + gp);
        phase_b((u % C::NVBUF) * C::TILEB);
        slot_end();
      };
      int i = 0;
      for (; i + C::NKBUF <= n; i += C::NKBUF)
#pragma unroll
        for (int u = 0; u < C::NKBUF; ++u) pp_step(i + u, u);
      for (; i < n; ++i) pp_step(i, i % C::NKBUF);
      if (gp == 0) {  // group 0 ends one slot early
        slot_loads(2 * n);
        slot_end();
      }
    }
  } else {
    if (te > tb) {
      pair_seek(pc, tb);
      fetch_pair(pc, kl, vl);
      if (te - tb > 1) fetch_pair(pc, kl + C::TILEB, vl + C::TILEB);
      load_q();  // its wait for Q also covers the tile loads issued before it
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (wave_active) {
        qk(0, sa);
        row_max(sa, mx);
      }
      __syncthreads();  // every wave is done with K(0): its buffer may be refilled
    }
    // step i of the unit uses K buffer i % 2 and V buffer i % 3; six steps per iteration
    // make every buffer offset a constant of its step (an LDS read address is then the
    // lane's offset register plus an immediate), the remainder takes them at run time
    auto step_i = [&](int t, int i) {
      const int cur = (i & 1) * C::TILEB, nxt = C::TILEB - cur;
      const int v3 = i % 3;
      const int vc = v3 * C::TILEB, vd = (v3 == 0 ? 2 : v3 - 1) * C::TILEB;
      step(t, sa, sb, mx, nxt, vc, kl + cur, vl + vd);
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sa[kb][qb] = sb[kb][qb];
    };
    int t = tb;
    for (; t + 6 <= te; t += 6)
#pragma unroll
      for (int i = 0; i < 6; ++i) step_i(t + i, i);
    for (; t < te; ++t) step_i(t, t - tb);
  }

  // ---- split part: this part's record (O / l, then m and l per row, all fp32) for
  // merge_kernel
  if (w.split_n > 1) {
    char* const records = (char*)hdr + ldc(hdr, kHdrRecordsOff);
    const int64_t rec_bytes = ldc(hdr, kHdrRecBytes);
    const int64_t ml_off = (int64_t)C::BQ * D * 4;  // m [BQ] then l [BQ]
    char* const mine = records + (int64_t)(w.rec0 + w.split_s) * rec_bytes;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int row = (wave * QB + qb) * 16 + l16;
      if (row >= w.qcount) continue;
      const float l = lsum[qb][0];
      const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
      for (int db = 0; db < C::NDB; ++db)
        *(f32x4*)(mine + ((int64_t)row * D + db * 16 + g * 4) * 4) = o[db][qb] * inv;
      if (g == 0) {
        ((float*)(mine + ml_off))[row] = m_i[qb];
        ((float*)(mine + ml_off))[C::BQ + row] = l;
      }
    }
    return;
  }

  // ---- epilogue: O /= l (l == 0 -> 1), store valid rows
  char* obase = (char*)p.o;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l = lsum[qb][0];
    const float inv = l > 0.f ? 1.f / l : 1.f;
    const int row = (wave * QB + qb) * 16 + l16;
    if (row >= w.qcount) continue;
    if (p.lse && g == 0) store_lse(p, w.h, w.q0, w.qpos0 + row, m_i[qb], l);
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
// MLA kernel for a 512-wide latent (K = V = one latent row shared by all heads), whole
// rows per wave: 8 waves x 16 query rows = 128 rows of one head share every 64-key latent
// tile loaded into LDS.  Filling those 64 KiB tiles is what bounds an MLA kernel (a
// workgroup of 64 rows that splits the 512 columns over its waves spent ~20% of its time
// on them), so the rows per tile matter more than anything else.  Wave w owns rows
// [16w, 16w+16) end to end: S^T for all 64 keys over the full 512-wide dot product (Q in
// registers), the online softmax in its own lanes, and O^T for all 512 columns (128
// accumulator registers), so the waves never exchange scores.  K = V: one tile feeds the
// b128 K reads of S^T and the tr16 V reads of O^T, with the pipelined kernel's swizzle
// (kv_swz).  Both MFMA phases read their LDS fragments LEAD slots ahead, in fenced slots
// (at ~246 VGPRs the compiler would otherwise read each fragment just before its MFMA).
// ---------------------------------------------------------------------------
struct MlaRowsCfg {
  static constexpr int D = 512;
  static constexpr int NW = 8;
  static constexpr int NT = NW * 64;
  static constexpr int BQ = NW * 16;       // query rows per workgroup
  static constexpr int BK = 64;            // keys per tile
  static constexpr int ROWB = D * 2;
  static constexpr int TILEB = BK * ROWB;  // 64 KiB
  static constexpr int KC = D / 32;        // 32-wide contraction steps of S^T
  static constexpr int NDB = D / 16;       // 16-column blocks of O^T
  static constexpr int NKB = BK / 16;      // 16-key blocks of S^T
  static constexpr int NKS = BK / 32;      // 32-key steps of O^T
  static constexpr int LDS_BYTES = 2 * TILEB;
};

template <typename T, bool PAGED, bool LSE>
__global__ __launch_bounds__(MlaRowsCfg::NT, 1) void attn_mla_rows_kernel(
    const fmlm_attn_params p, const int4* __restrict__ units, const int32_t* __restrict__ hdr) {
  typedef MlaRowsCfg C;
  typedef typename Mfma<T>::v8 v8;
  constexpr int D = C::D, BK = C::BK;
  extern __shared__ __align__(16) char smem_raw[];

  // packed calls use head-packed tiles: 128 consecutive rows of the sequence's H*len
  // (head, position) rows, all heads reading the same latent
  const bool hpack = p.cu_seqlens_q != nullptr;
  // the grid covers the queue slots (8 * cap workgroups), workgroup w taking entry w / 8
  // of queue w % 8: a sequence's tiles stay on the XCDs the schedule put them on
  const int u = hpack ? queue_first(hdr, blockIdx.x) : (int)blockIdx.x;
  WorkItem w;
  if (u < 0 || !resolve_work(p, units, u, C::BQ, w, hpack)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int row = wave * 16 + l16;  // the query row of this lane's S^T / O^T column
  const bool wave_active = wave * 16 < w.qcount;
  // element offsets of this lane's q and o rows
  int64_t q_off, o_off;
  {
    int hq = w.h, pq = w.qpos0 + row;
    if (hpack && w.len > 0) {
      hq = pq / w.len;
      pq -= hq * w.len;
    }
    q_off = p.q_layout == FMLM_LAYOUT_PACKED ? (int64_t)hq * p.q_sh + (int64_t)(w.q0 + pq) * p.q_sn
                                             : (int64_t)w.b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)pq * p.q_sn;
    o_off = p.o_layout == FMLM_LAYOUT_PACKED ? (int64_t)hq * p.o_sh + (int64_t)(w.q0 + pq) * p.o_sn
                                             : (int64_t)w.b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)pq * p.o_sn;
  }

  // ---- Q^T fragments (B operand of S^T = K Q^T) for step kc, as stored but for the
  // sign of a negative scale.  Scores in log2 units are c * (K Q^T), c = |scale|*log2(e),
  // applied in fp32 by the FMA that subtracts the running max (as the reference scales
  // the fp32 product; a Q pre-scaled in the input type would round each q*c to 8 bits at
  // bf16).  The floor keeps -inf * c == -inf for masked keys at scale 0.
  const uint32_t qsign = p.scale < 0.f ? 0x80008000u : 0u;
  const float c = fmaxf(fabsf(p.scale) * kLog2e, 1e-30f);
  v8 qf[C::KC];
  {
    const bool ok = row < w.qcount;
    const char* src = (const char*)p.q + q_off * 2;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      u32x4 raw = u32x4{0u, 0u, 0u, 0u};
      if (ok) raw = *(const u32x4*)(src + (kc * 32 + g * 8) * 2);
      qf[kc] = __builtin_bit_cast(v8, raw ^ qsign);
    }
  }
  // ---- per-lane LDS offsets (kv_swz layout, 1 KiB rows): the K fragment of block kb,
  // step kc is at (kk ^ 64*(kc%4)) + kb*16*ROWB + 256*(kc/4); the V tr16 fragment of step
  // ks, column block db, half h at (vv ^ 32*(db%8)) + (32 ks + 16 h)*ROWB + 256*(db/8).
  // The XOR terms select the swizzled 16-byte chunk; they touch bits 5..7 only, which the
  // row and stage offsets leave clear.  kv_swz serves both read shapes of the tile (b128
  // K fragments, tr16 V fragments) without bank conflicts.
  int kk, vv;
  {
    const int ksw = kv_swz<D>(l16);
    kk = l16 * C::ROWB + 64 * (ksw >> 2) + 16 * (g ^ (ksw & 3));
    const int vr = 4 * g + (l16 >> 2);
    const int vsw = kv_swz<D>(vr);
    const int x = (l16 & 3) >> 1;
    vv = vr * C::ROWB + 32 * (vsw >> 1) + 16 * (x ^ (vsw & 1)) + 8 * (l16 & 1);
  }
  // LDS fragment reads in flight ahead of their MFMA (the paged variant keeps its page
  // window in registers, which the longer lead would spill)
  constexpr int LEAD = PAGED ? 2 : 3;

  const int nt0 = (w.seg[0].n + BK - 1) / BK;
  const int nt1 = (w.seg[1].n + BK - 1) / BK;
  const int ntiles = nt0 + nt1;
  PageWindow pwin;  // paged context: page ids of the tiles around the last one fetched
  page_window_reset(pwin);

  // ---- direct loads of tile t into stage st: wave w brings rows w + 8j, one 1 KiB row
  // per load; lane l fetches logical chunk l ^ kv_swz(row), which lands in physical chunk
  // l.  Rows past a segment end repeat its last row (their scores are masked).  Issued
  // from inline asm like the pipelined kernel's loads; the wait + barrier at the end of
  // each tile orders them.
  auto fetch = [&](int t, int st) {
    const int sg = t < nt0 ? 0 : 1;
    const KvSeg& s = w.seg[sg];
    const int tt = sg == 0 ? t : t - nt0;
    const int j0 = tt * BK;
    const int last = __builtin_amdgcn_readfirstlane(s.n - 1);
    const uint32_t lds0 = lds_addr(smem_raw + st * C::TILEB);
    // paged segments (the context): tile tt is one page; rows are relative to its row 0
    const char* base = s.k + s.kbase * 2;
    int kb0 = j0;
    if constexpr (PAGED) {
      if (sg == 0 && w.seg[0].pages) {
        base = page_row0(w.seg[0], base, tt, pwin);
        kb0 = 0;
      }
    }
#pragma unroll
    for (int j = 0; j < BK / C::NW; ++j) {
      const int r = wave + j * C::NW;
      const int key = min(j0 + r, last) - j0 + kb0;
      dma16_sbase(uniform_ptr(base + (int64_t)key * s.ksn * 2), (uint32_t)((lane ^ kv_swz<D>(r)) << 4),
                  __builtin_amdgcn_readfirstlane(lds0 + r * C::ROWB));
    }
  };

  f32x4 o[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i = -INFINITY, l_i = 0.f;

  if (ntiles > 0) fetch(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const char* tile = smem_raw + (t & 1) * C::TILEB;
    // a wave with query rows loads its share of tile t+1 once its S MFMAs have read tile
    // t's K fragments (the DMA writes into LDS then overlap the P V phase rather than the
    // b128 fragment reads of S; measured 2.6-3.3% faster at config 5 than loading at the
    // top of the tile, and faster than any later point, which leaves the loads less time)
    if (!wave_active && t + 1 < ntiles) fetch(t + 1, (t + 1) & 1);
    if (wave_active) {
      // Four phases of 32 fenced slots: slot f issues the LDS read of fragment f + LEAD
      // and the MFMA of fragment f.  K fragments f < 64 build S^T: half h = f / 32 covers
      // key blocks 2h, 2h+1 (f = 32 h + 2 kc + kb % 2).  V fragments f = 64 + 32 ks + db
      // build O^T from the P of key step ks.  Half 0's softmax runs beside half 1's S
      // MFMAs, half 1's beside the key-step-0 P V MFMAs, so no phase waits on exp.
      const uint32_t ktile = lds_addr(tile) + kk;
      const uint32_t vtile = lds_addr(tile) + vv;
      auto fread = [&](int f) -> v8 {
        if (f < 64) {
          const int kc = (f & 31) >> 1, kb = 2 * (f >> 5) + (f & 1);
          const uint32_t a = (ktile ^ (64 * (kc & 3))) + kb * 16 * C::ROWB + 256 * (kc >> 2);
          return *(const FMLM_LDS v8*)(uintptr_t)a;
        }
        const int ks = (f - 64) >> 5, db = (f - 64) & 31;
        const uint32_t a = (vtile ^ (32 * (db & 7))) + ks * 32 * C::ROWB + 256 * (db >> 3);
        const s16x4 lo = lds_read_tr16_at(a);
        const s16x4 hi = lds_read_tr16_at(a + 16 * C::ROWB);
        return __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      };
      const int nk = t < nt0 ? min(BK, w.seg[0].n - t * BK) : min(BK, w.seg[1].n - (t - nt0) * BK);
      f32x4 s[C::NKB];
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) s[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      u32x4 pf[C::NKS];  // P^T of key step ks: element (kb&1)*4 + r is key 32 ks + 16 (kb&1) + 4g + r
      // P of key block kb, keys 4g + r and 4g + r + 1 (r even), against the running max
      auto exp_pair = [&](int kb, int r, bool add_l) {
        if (r == 0) pin(s[kb]);
        f32x2 x = f32x2{fast_exp2(fmaf(s[kb][r], c, -m_i)), fast_exp2(fmaf(s[kb][r + 1], c, -m_i))};
        if (add_l) l_i += x[0] + x[1];
        uint32_t wv = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, typename Pair<T>::type));
        pin(wv);
        pf[kb >> 1][(kb & 1) * 2 + (r >> 1)] = wv;
      };
      // softmax bookkeeping of half h once its MFMAs are done: mask keys past the tile's
      // end, row max (lane-local, then over the 4 lanes of the row), lazy rescale.  When
      // half 1 raises the maximum, half 0's P (already computed) is rescaled like O and
      // l_i, which holds half 0's sums.
      auto half_check = [&](int h) {
        if (nk < BK) {
          const int lim = nk - 4 * g;  // key kb*16 + 4g + r is valid iff kb*16 + r < lim
#pragma unroll
          for (int kb = 2 * h; kb < 2 * h + 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (kb * 16 + r >= lim) s[kb][r] = -INFINITY;
        }
        float mx = vmax(vmax(vmax(s[2 * h][0], s[2 * h][1]), vmax(s[2 * h][2], s[2 * h][3])),
                        vmax(vmax(s[2 * h + 1][0], s[2 * h + 1][1]), vmax(s[2 * h + 1][2], s[2 * h + 1][3])));
        mx = lane_max_xor16_32(mx) * c;  // log2 units (c > 0)
        const bool grow = mx > m_i + kRescaleSlack;
        if (__builtin_amdgcn_ballot_w64(grow)) {
          const float m_new = grow ? mx : m_i;
          const float alpha = fast_exp2(m_i - m_new);  // 1 where unchanged, 0 on the first tile
          m_i = m_new;
          l_i *= alpha;
#pragma unroll
          for (int db = 0; db < C::NDB; ++db) o[db] *= alpha;
          if (h == 1)  // half 0's P, computed against the old maximum
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // element e through a local: a __builtin_bit_cast of the vector element
              // itself compiles (clang of ROCm 7.2) to a read of element 0
              const uint32_t u = pf[0][e];
              typename Pair<T>::type v = __builtin_bit_cast(typename Pair<T>::type, u);
              const f32x2 x = __builtin_convertvector(v, f32x2) * alpha;
              pf[0][e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, typename Pair<T>::type));
            }
        }
      };
      constexpr int NF = 128;
      v8 fr[LEAD + 1];
#pragma unroll
      for (int r = 0; r < LEAD; ++r) fr[r] = fread(r);
      auto slot = [&](const int f) {
        if (f + LEAD < NF) fr[(f + LEAD) % (LEAD + 1)] = fread(f + LEAD);
        const v8 a = fr[f % (LEAD + 1)];
        if (f < 64) {
          const int kb = 2 * (f >> 5) + (f & 1);
          s[kb] = Mfma<T>::run(a, qf[(f & 31) >> 1], s[kb]);
          // half 0's P beside half 1's S MFMAs: one exp pair every 8 slots
          if (f >= 32 && (f & 7) == 7) {
            const int q = (f - 32) >> 3;
            exp_pair(q >> 1, (q & 1) * 2, true);
          }
        } else {
          const int ks = (f - 64) >> 5, db = (f - 64) & 31;
          o[db] = Mfma<T>::run(a, __builtin_bit_cast(v8, pf[ks]), o[db]);
          // half 1's P beside the key-step-0 P V MFMAs (done before step 1 starts)
          if (ks == 0 && (db & 7) == 3) {
            const int q = db >> 3;
            exp_pair(2 + (q >> 1), (q & 1) * 2, true);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      };
      // four unrolled phases of 32 slots (one 128-slot loop is too large to unroll)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int f = 0; f < 32; ++f) slot(f);
      __builtin_amdgcn_s_setprio(0);
      half_check(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int f = 32; f < 64; ++f) slot(f);
      __builtin_amdgcn_s_setprio(0);
      if (t + 1 < ntiles) fetch(t + 1, (t + 1) & 1);
      half_check(1);
      __builtin_amdgcn_s_setprio(2);
#pragma unroll
      for (int f = 64; f < 96; ++f) slot(f);
#pragma unroll
      for (int f = 96; f < 128; ++f) slot(f);
      __builtin_amdgcn_s_setprio(0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // tile t+1 landed
    __syncthreads();                // and every wave is done with tile t
  }

  // ---- epilogue: l over the 4 lanes holding the row's keys, O /= l, store the row
  l_i += __shfl_xor(l_i, 16);
  l_i += __shfl_xor(l_i, 32);
  if (row < w.qcount) {
    const float inv = l_i > 0.f ? 1.f / l_i : 1.f;
    char* dst = (char*)p.o + o_off * 2;
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      T v4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = (T)(o[db][r] * inv);
      *(u32x2*)(dst + (db * 16 + g * 4) * 2) = *(const u32x2*)v4;
    }
    // the row statistic (LSE instantiation only: the row and the sequence ranges it needs
    // cost the kernel, at 256 VGPRs, registers across the tile loop), after the row's
    // store: its (head, position) as for the q and o offsets
    if (LSE && p.lse && g == 0) {
      int rr = row;
      asm volatile("" : "+v"(rr));
      int hq = w.h, pq = w.qpos0 + rr;
      if (hpack && w.len > 0) {
        hq = pq / w.len;
        pq -= hq * w.len;
      }
      store_lse(p, hq, w.q0, pq, m_i, l_i);
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
  static constexpr int TPR = D / 4 < 16 ? D / 4 : 16;  // threads per query row
  static constexpr int DPT = D / TPR;                   // dims per thread (a multiple of 4)
  static constexpr int NT = 256;
  static constexpr int RPW = NT / TPR;                  // query rows per workgroup
  static constexpr int BKS = 4096 / D < 64 ? 4096 / D : 64;  // keys per LDS tile
  static constexpr int LDS_BYTES = 2 * BKS * D * 4;
  static_assert(DPT % 4 == 0 && (TPR & (TPR - 1)) == 0, "simt tiling");
};

template <typename T>
FMLM_DEV float to_f(T x) {
  return (float)x;
}

// four consecutive elements as floats
template <typename T>
FMLM_DEV float4 load4(const T* p) {
  return float4{to_f(p[0]), to_f(p[1]), to_f(p[2]), to_f(p[3])};
}
template <>
FMLM_DEV float4 load4<float>(const float* p) {
  return *(const float4*)p;
}

// fp32 (and head dims without an MFMA instantiation): TPR threads per query row, each
// holding DPT dims of q and o; a row's partial dot products meet through xor shuffles
// inside its TPR lanes.  K/V tiles of BKS keys are staged as fp32 in LDS and read as
// float4 (a row's lanes cover one contiguous key row).
template <typename T, int D>
__global__ __launch_bounds__(SimtCfg<D>::NT) void attn_simt_kernel(
    const fmlm_attn_params p, const int4* __restrict__ units, const int32_t* __restrict__ hdr) {
  typedef SimtCfg<D> C;
  extern __shared__ __align__(16) char smem_raw[];
  float* Kf = (float*)smem_raw;
  float* Vf = Kf + C::BKS * D;

  const int u = p.cu_seqlens_q ? workgroup_unit(hdr) : (int)blockIdx.x;
  WorkItem w;
  if (u < 0 || !resolve_work(p, units, u, C::RPW, w)) return;
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
  for (int d = 0; d < C::DPT; d += 4) {
    const float4 v4 = ok ? load4(qp + d) : float4{0.f, 0.f, 0.f, 0.f};
    q[d] = v4.x;
    q[d + 1] = v4.y;
    q[d + 2] = v4.z;
    q[d + 3] = v4.w;
    o[d] = o[d + 1] = o[d + 2] = o[d + 3] = 0.f;
  }
  float m_i = -INFINITY, l_i = 0.f;

  // the two segments unrolled: a run-time index into w.seg would put w in scratch memory
#pragma unroll
  for (int si = 0; si < 2; ++si) {
    const KvSeg& s = w.seg[si];
    for (int j0 = 0; j0 < s.n; j0 += C::BKS) {
      const int nk = min(C::BKS, s.n - j0);
      __syncthreads();
      for (int e = tid * 4; e < C::BKS * D; e += C::NT * 4) {
        const int kk = e / D, d = e % D;
        float4 kv = float4{0.f, 0.f, 0.f, 0.f}, vv = kv;
        if (kk < nk) {
          kv = load4((const T*)s.k + seg_row(s, j0 + kk, false, cu, B) + d);
          vv = load4((const T*)s.v + seg_row(s, j0 + kk, true, cu, B) + d);
        }
        *(float4*)(Kf + e) = kv;
        *(float4*)(Vf + e) = vv;
      }
      __syncthreads();
      float sc[C::BKS];
      float mx = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < C::BKS; ++kk) {
        float acc = 0.f;
#pragma unroll
        for (int d = 0; d < C::DPT; d += 4) {
          const float4 k4 = *(const float4*)(Kf + kk * D + d0 + d);
          acc += q[d] * k4.x + q[d + 1] * k4.y + q[d + 2] * k4.z + q[d + 3] * k4.w;
        }
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
        for (int d = 0; d < C::DPT; d += 4) {
          const float4 v4 = *(const float4*)(Vf + kk * D + d0 + d);
          o[d] += pr * v4.x;
          o[d + 1] += pr * v4.y;
          o[d + 2] += pr * v4.z;
          o[d + 3] += pr * v4.w;
        }
      }
    }
  }
  if (!ok) return;
  const float inv = l_i > 0.f ? 1.f / l_i : 1.f;
  if (p.lse && part == 0) store_lse(p, w.h, w.q0, w.qpos0 + row, m_i, l_i);
  T* op = (T*)p.o + w.o_row0 + (int64_t)row * w.o_sn + d0;
#pragma unroll
  for (int d = 0; d < C::DPT; ++d) op[d] = (T)(o[d] * inv);
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// Split-KV merge: for every split group (query tile (b, h, tile) whose key range was
// cut into S parts), O = sum_s 2^(m_s - M) l_s O_s / sum_s 2^(m_s - M) l_s with
// M = max_s m_s, over the parts' records (O_s = part output / l_s as fp32, m_s in log2
// units, l_s its row sum), so the merged row is rounded to the output type once, as an
// unsplit row is.  Grid-stride over groups; 8 columns of a row per thread.
// ---------------------------------------------------------------------------
constexpr int kMergeRows = 128;  // largest split-capable query tile

template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(const fmlm_attn_params p, int BQ,
                                                    const int32_t* __restrict__ header) {
  typedef typename Mfma<T>::v8 v8;
  __shared__ float s_w[kMergeRows][kMaxSplits];  // per row: part weights / their sum
  const int n_groups = header[kHdrGroups];
  const int4* groups = (const int4*)((const char*)header + header[kHdrGroupsOff]);
  const char* records = (const char*)header + header[kHdrRecordsOff];
  const int64_t rec_bytes = header[kHdrRecBytes];
  const int D = p.D;
  const int64_t ml_off = (int64_t)BQ * D * 4;
  for (int gi = blockIdx.x; gi < n_groups; gi += gridDim.x) {
    const int4 gr = groups[gi];
    const int b = gr.x, h = gr.y & 0xffff, tile = (int)((uint32_t)gr.y >> 16), S = gr.w;
    if (b < 0 || b >= p.B || h >= p.H) continue;
    const SeqInfo si = seq_info(p, b);
    const int qcount = min(BQ, si.len - tile * BQ);
    const int64_t ob = p.o_layout == FMLM_LAYOUT_PACKED
                           ? (int64_t)h * p.o_sh + (int64_t)si.q0 * p.o_sn
                           : (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
    const int64_t o_row0 = ob + (int64_t)tile * BQ * p.o_sn;
    const char* rec0 = records + (int64_t)gr.z * rec_bytes;
    // weights of row r: 2^(m_s - M) l_s / sum, all parts' (m, l) loaded at once
    for (int r = threadIdx.x; r < qcount; r += blockDim.x) {
      float m[kMaxSplits], l[kMaxSplits];
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp) {
        const float* ml = (const float*)(rec0 + (sp < S ? sp : 0) * rec_bytes + ml_off);
        m[sp] = sp < S ? ml[r] : -INFINITY;
        l[sp] = sp < S ? ml[BQ + r] : 0.f;
      }
      float M = -INFINITY;
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp) M = fmaxf(M, m[sp]);
      float L = 0.f;
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp) {
        l[sp] = M == -INFINITY ? 0.f : fast_exp2(m[sp] - M) * l[sp];
        L += l[sp];
      }
      const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp) s_w[r][sp] = l[sp] * inv;
      if (p.lse) store_lse(p, h, si.q0, tile * BQ + r, M, L);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < qcount * (D / 8); idx += blockDim.x) {
      const int row = idx / (D / 8), c8 = idx - row * (D / 8);
      const char* src = rec0 + ((int64_t)row * D + c8 * 8) * 4;
      f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll 4
      for (int sp = 0; sp < S; ++sp) {
        const f32x4 x0 = *(const f32x4*)(src + sp * rec_bytes);
        const f32x4 x1 = *(const f32x4*)(src + sp * rec_bytes + 16);
        const float ws = s_w[row][sp];
        a0 += ws * x0;
        a1 += ws * x1;
      }
      v8 res;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        res[e] = (T)a0[e];
        res[4 + e] = (T)a1[e];
      }
      *(v8*)((char*)p.o + (o_row0 + (int64_t)row * p.o_sn + c8 * 8) * 2) = res;
    }
    __syncthreads();  // s_w is rewritten for the next group
  }
}

struct Launch {
  int bq;         // query rows per workgroup
  int threads;
  int lds;
  const void* fn;
  bool split = false;  // kernel can run split-KV units
  bool hpack = false;  // packed tiles span (head, position) rows (MLA: one latent for all heads)
  bool paged = false;  // kernel reads a paged context (key tile = FMLM_PAGE_ROWS rows)
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

template <typename T, int D, int QB, int NW, int BK, int PPB = 0>
static Launch mfma3_launch(bool paged) {
  typedef Mfma3Cfg<T, D, QB, NW, BK, PPB> C;
  static_assert(BK == kSplitBK, "split planning assumes the kernel's key tile");
  static_assert(BK == FMLM_PAGE_ROWS, "a paged context tile is one page");
  const void* fn = (const void*)&attn_mfma3_kernel<T, D, QB, NW, BK, false, PPB>;
  if constexpr (PPB == 0) {
    if (paged) fn = (const void*)&attn_mfma3_kernel<T, D, QB, NW, BK, true, PPB>;
  } else if (paged) {  // the ping-pong configurations read contiguous contexts only
    fn = nullptr;
  }
  return Launch{C::BQ, C::NT, C::LDS_BYTES, fn, true, false, true};
}

// the paged instantiation only for paged contexts: the page lookup costs registers the
// contiguous kernel (at 256 VGPRs) does not have; the LSE one only for calls that store
// the row statistics
template <typename T>
static Launch mla_rows_launch(bool paged, bool lse) {
  static_assert(MlaRowsCfg::BK == FMLM_PAGE_ROWS, "a paged context tile is one page");
  const void* fn = paged ? (lse ? (const void*)&attn_mla_rows_kernel<T, true, true>
                                : (const void*)&attn_mla_rows_kernel<T, true, false>)
                         : (lse ? (const void*)&attn_mla_rows_kernel<T, false, true>
                                : (const void*)&attn_mla_rows_kernel<T, false, false>);
  return Launch{MlaRowsCfg::BQ, MlaRowsCfg::NT, MlaRowsCfg::LDS_BYTES, fn, false, true, true};
}

// MFMA kernels by head dim.  The pipelined kernel and the 512-wide latent kernel need
// linear main-key addressing; causal_query_seq_attn over padded K/V (a per-row sequence
// lookup) takes the register-staged kernel.  The latent kernel also needs K = V (MLA).
template <typename T>
static bool pick_mfma(const fmlm_attn_params& p, Launch& L) {
  const bool lookup = (p.flags & FMLM_FLAG_CAUSAL_SEQ) && p.cu_seqlens_q &&
                      p.kv_layout != FMLM_LAYOUT_PACKED;
  if (lookup) {
    if (p.tile_config > 1) return false;
    switch (p.D) {
      case 16: L = mfma_launch<T, 16, 2, 4, 64>(); return true;
      case 32: L = mfma_launch<T, 32, 2, 4, 64>(); return true;
      case 64: L = mfma_launch<T, 64, 2, 4, 64>(); return true;
      case 128: L = mfma_launch<T, 128, 2, 4, 64>(); return true;
      case 256: L = mfma_launch<T, 256, 1, 4, 64>(); return true;
      default: return false;
    }
  }
  const bool paged = p.ctx_block_table != nullptr;
  // The library's choice (tile_config 0).  At D = 64 and 128, 64-row workgroups (one
  // 16-row block per wave) when the sequences average at most 64 query rows: a 128-row
  // workgroup would then leave half its waves without rows, one working wave per SIMD.
  // Measured 19-28% faster for 16-64 rows per sequence against a shared context, level at
  // 48-80 rows or where per-sequence contexts make the launch HBM-bound, 12-20% slower
  // at 64-128 rows.  128-row workgroups (two blocks per wave) otherwise.
  const bool short_q = (int64_t)p.total_q <= 64LL * p.B;
  const int k = p.tile_config > 0 ? p.tile_config : ((p.D == 64 || p.D == 128) && short_q ? 3 : 1);
  switch (p.D) {
    case 16:
      if (k == 1) L = mfma3_launch<T, 16, 2, 4, 64>(paged); else return false;
      return true;
    case 32:
      if (k == 1) L = mfma3_launch<T, 32, 2, 4, 64>(paged); else return false;
      return true;
    case 64:
      if (k == 1) L = mfma3_launch<T, 64, 2, 4, 64>(paged);
      else if (k == 2) L = mfma3_launch<T, 64, 2, 8, 64>(paged);
      else if (k == 3) L = mfma3_launch<T, 64, 1, 4, 64>(paged);
      else if (k == 4) L = mfma3_launch<T, 64, 2, 8, 64, 3>(paged);
      else return false;
      return true;
    case 128:
      if (k == 1) L = mfma3_launch<T, 128, 2, 4, 64>(paged);
      else if (k == 2) L = mfma3_launch<T, 128, 2, 8, 64>(paged);
      else if (k == 3) L = mfma3_launch<T, 128, 1, 4, 64>(paged);
      else if (k == 4) L = mfma3_launch<T, 128, 1, 8, 64>(paged);
      else if (k == 5) L = mfma3_launch<T, 128, 2, 8, 64, 3>(paged);
      else return false;
      return true;
    case 256:
      if (k == 1) L = mfma3_launch<T, 256, 1, 4, 64>(paged);
      else if (k == 2) L = mfma3_launch<T, 256, 1, 8, 64>(paged);
      else return false;
      return true;
    case 512:
      if (!(p.flags & FMLM_FLAG_MLA) || k != 1) return false;
      L = mla_rows_launch<T>(p.ctx_block_table != nullptr, p.lse != nullptr);
      return true;
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

static int pick_launch(const fmlm_attn_params& p, Launch& L) {
  bool ok = false;
  if (p.tile_config < 0) return FMLM_E_ARG;
  switch (p.dtype) {
    case FMLM_DTYPE_BF16: ok = pick_mfma<bf16>(p, L) || (p.tile_config <= 1 && pick_simt<bf16>(p.D, L)); break;
    case FMLM_DTYPE_F16: ok = pick_mfma<f16>(p, L) || (p.tile_config <= 1 && pick_simt<f16>(p.D, L)); break;
    case FMLM_DTYPE_F32: ok = pick_simt<float>(p.D, L); break;
    default: return FMLM_E_DTYPE;
  }
  if (!ok) return p.tile_config > 1 ? FMLM_E_ARG : FMLM_E_HEAD_DIM;
  // a paged context needs a kernel whose key tile is one page (not fp32, not per-row
  // lookups), and a configuration with a paged instantiation
  if (p.ctx_block_table && !(p.flags & FMLM_FLAG_PREFILL) && !L.paged) return FMLM_E_ARG;
  if (!L.fn) return FMLM_E_ARG;
  return 0;
}

// Allow the kernel's dynamic LDS (> 64 KiB for some tiles), once per kernel.
static int allow_lds(const Launch& L) {
  static std::mutex mu;
  static const void* raised[64];
  static int n_raised = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_raised; ++i)
    if (raised[i] == L.fn) return 0;
  hipError_t e = hipFuncSetAttribute(L.fn, hipFuncAttributeMaxDynamicSharedMemorySize, L.lds);
  if (e != hipSuccess) return (int)e;
  if (n_raised < 64) raised[n_raised++] = L.fn;
  return 0;
}

// Resident workgroup slots of a kernel (CUs x workgroups per CU), once per kernel; 0 on
// a query error.
static int resident_slots(const Launch& L) {
  static std::mutex mu;
  static const void* fns[64];
  static int slots_of[64];
  static int n_fns = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_fns; ++i)
    if (fns[i] == L.fn) return slots_of[i];
  int dev = 0, cus = 0, per_cu = 0;
  if (allow_lds(L) != 0 || hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, L.fn, L.threads, L.lds) != hipSuccess)
    return 0;
  const int slots = cus * (per_cu > 0 ? per_cu : 1);
  if (n_fns < 64) {
    fns[n_fns] = L.fn;
    slots_of[n_fns++] = slots;
  }
  return slots;
}

// Split-KV sizing: the GPU's workgroup slots for this kernel, the record capacity and
// the record size.
struct SplitCfg {
  int slots = 0;
  int rec_cap = 0;        // 0: no split
  int64_t rec_bytes = 0;  // per record: rows x (D fp32 + m + l)
};

static SplitCfg split_cfg(const fmlm_attn_params& p, const Launch& L) {
  SplitCfg sc;
  if (!L.split || !p.cu_seqlens_q) return sc;
  sc.slots = resident_slots(L);
  if (sc.slots == 0) return sc;
  // every sequence's tiles but its last are full, so there are at least
  // H * (total_q - B*bq) / bq units: when that already fills kSplitRounds rounds, the
  // schedule cannot split (and no records or merge launch are needed)
  const int64_t min_units = (int64_t)p.H * (((int64_t)p.total_q - (int64_t)p.B * L.bq) / L.bq);
  if (min_units >= (int64_t)(kSplitRounds * sc.slots) || L.bq > kMergeRows) return SplitCfg{};
  sc.rec_cap = 3 * sc.slots;
  sc.rec_bytes = ((int64_t)L.bq * (p.D * 4 + 8) + 15) / 16 * 16;
  return sc;
}

// Units of a dense call: slots of 8 XCDs x ceil(B*H / 8) groups x ceil(N / bq) tiles.
static int64_t dense_units(const fmlm_attn_params& p, int bq) {
  return (int64_t)kXcds * (((int64_t)p.B * p.H + kXcds - 1) / kXcds) * ((p.N + bq - 1) / bq);
}

// Entries per queue of a packed call: a bound on the launch's units, so that one queue
// can take all of them whatever the placement.  Sequence b has ceil(L_b / bq) <= L_b / bq
// + 1 query tiles per head (head-packed: ceil(H L_b / bq) in all); with splits, which
// happen only below kSplitRounds * slots unsplit units, add every split part.
static int64_t queue_cap(const fmlm_attn_params& p, int bq, const SplitCfg& sc, bool hpack) {
  int64_t units = hpack ? ((int64_t)p.H * p.total_q + bq - 1) / bq + p.B
                        : (int64_t)p.H * (((int64_t)p.total_q + bq - 1) / bq + p.B);
  if (sc.rec_cap > 0) {
    const int64_t split_units = (int64_t)(kSplitRounds * sc.slots) + 1 + sc.rec_cap;
    units = split_units > units ? split_units : units;
  }
  return units;
}

// Grid (one unit per workgroup): a dense call's slots; cap workgroups for a packed call
// (spares take what overflows a queue's static entries), 8 * cap head-packed.
static int64_t grid_size(const fmlm_attn_params& p, const Launch& L, const SplitCfg& sc) {
  if (!p.cu_seqlens_q) return dense_units(p, L.bq);
  const int64_t cap = queue_cap(p, L.bq, sc, L.hpack);
  return L.hpack ? kXcds * cap : cap;
}

// Schedule buffer layout (see schedule_kernel): header, 8 queues, groups, records.
struct SchedLayout {
  int64_t cap, units_off, groups_off, records_off, bytes;
};

static SchedLayout sched_layout(const fmlm_attn_params& p, int bq, const SplitCfg& sc, bool hpack) {
  SchedLayout l;
  l.cap = queue_cap(p, bq, sc, hpack);
  l.units_off = 256;
  l.groups_off = l.units_off + kXcds * l.cap * (int64_t)sizeof(int4);
  l.groups_off = (l.groups_off + 255) / 256 * 256;
  l.records_off = l.groups_off + (int64_t)sc.rec_cap * (int64_t)sizeof(int4);
  l.records_off = (l.records_off + 255) / 256 * 256;
  l.bytes = l.records_off + (int64_t)sc.rec_cap * sc.rec_bytes;
  return l;
}

static int64_t workspace_for(const fmlm_attn_params& p, const Launch& L) {
  if (!p.cu_seqlens_q) return 0;
  return sched_layout(p, L.bq, split_cfg(p, L), L.hpack).bytes;
}

static int check_params(const fmlm_attn_params& p) {
  if (p.B < 0 || p.H < 0 || p.N < 0 || p.D < 1 || p.total_q < 0 || p.ctx_len < 0) return FMLM_E_ARG;
  // row strides are applied as 32-bit offsets within a key tile
  const int64_t kMaxRowStride = 1 << 22;
  for (int64_t sn : {p.k_sn, p.v_sn, p.c_sn, p.q_sn, p.o_sn})
    if (sn < 0 || sn >= kMaxRowStride) return FMLM_E_ARG;
  if (!p.q || !p.o || !p.k || (!(p.flags & FMLM_FLAG_MLA) && !p.v)) return FMLM_E_ARG;
  if ((p.flags & FMLM_FLAG_CAUSAL_SEQ) && !p.cu_seqlens_q) return FMLM_E_ARG;
  if (!(p.flags & FMLM_FLAG_PREFILL)) {
    const bool has_ctx = p.cu_seqlens_kv || p.ctx_len > 0;
    if (has_ctx && !p.cu_seqlens_kv && p.ctx_len > 0 && !p.k_ctx) return FMLM_E_ARG;
    if ((p.cu_seqlens_kv || p.ctx_index) && p.ctx_batch < 1) return FMLM_E_ARG;
    if (p.ctx_block_table && (p.ctx_pages_per_batch < 0 || p.ctx_rows < 1 || p.ctx_page_stride < 0 ||
                              p.ctx_batch < 1 || !p.k_ctx))
      return FMLM_E_ARG;
  }
  return 0;
}

static int launch_schedule(const fmlm_attn_params& p, const Launch& L, const SplitCfg& sc, char* sched,
                           hipStream_t s) {
  const SchedLayout l = sched_layout(p, L.bq, sc, L.hpack);
  // the unit's 16-bit tile field: tiles of N rows, or of H*N (H*total_q) rows head-packed;
  // queue entries are addressed with 32-bit indices
  const int64_t rows = L.hpack ? (int64_t)p.H * (p.N > 0 ? p.N : p.total_q) : p.N;
  if (kXcds * l.cap > 0x7fffffff || p.H > 0xffff || (rows + L.bq - 1) / L.bq > 0xffff) return FMLM_E_ARG;
  int32_t* header = (int32_t*)sched;
  hipLaunchKernelGGL(schedule_kernel, dim3(1), dim3(kSchedThreads), 0, s, p, L.bq, (int)l.cap,
                     sc.slots, sc.rec_cap, (int4*)(sched + l.units_off), header,
                     (int4*)(sched + l.groups_off), (int)l.groups_off, (int)l.records_off,
                     (int)sc.rec_bytes, (int)L.hpack);
  return launch_status();
}

// The attention launch (plus the split merge) over the schedule at `sched`, which is
// built first when `build` is set.  sc must be the split sizing the schedule was (or is)
// built with.
static int launch_attention(const fmlm_attn_params& p, const Launch& L, const SplitCfg& sc, char* sched,
                            bool build, hipStream_t s) {
  int rc = allow_lds(L);
  if (rc) return rc;
  int4* units = nullptr;
  int32_t* header = nullptr;
  if (p.cu_seqlens_q) {
    header = (int32_t*)sched;
    units = (int4*)(sched + 256);
    if (build) {
      rc = launch_schedule(p, L, sc, sched, s);
      if (rc) return rc;
    }
  }
  const int64_t gx = grid_size(p, L, sc);
  if (gx <= 0) return 0;
  if (gx > 0x7fffffff) return FMLM_E_ARG;
  fmlm_attn_params pc = p;
  void* args[] = {(void*)&pc, (void*)&units, (void*)&header};
  hipError_t e = hipLaunchKernel(L.fn, dim3((unsigned)gx), dim3(L.threads), args, (size_t)L.lds, s);
  if (e != hipSuccess) return (int)e;
  if (sc.rec_cap > 0) {  // split groups (if the schedule made any) are merged here
    const dim3 mg((unsigned)(sc.rec_cap < 1024 ? sc.rec_cap : 1024));
    if (p.dtype == FMLM_DTYPE_BF16)
      hipLaunchKernelGGL(merge_kernel<bf16>, mg, dim3(256), 0, s, p, L.bq, (const int32_t*)header);
    else
      hipLaunchKernelGGL(merge_kernel<f16>, mg, dim3(256), 0, s, p, L.bq, (const int32_t*)header);
  }
  return launch_status();
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point: the schedule (header, units, split groups)
// and the split records live in this library-owned array, one copy per GPU, instead of
// a caller's workspace.  Host code never uses the array's name as an address: it reads
// each device's address once with hipGetSymbolAddress (scratch_on_current_device).
// Every call on a GPU reuses that GPU's array; calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchBytes = FMLM_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

static int scratch_on_current_device(char** out) {
  static std::mutex mu;
  static char* ptrs[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return FMLM_E_ARG;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return FMLM_E_ARG;
    ptrs[dev] = (char*)ptr;
  }
  *out = ptrs[dev];
  return 0;
}

// The split sizing of the allocation-free path: as split_cfg, with the record count cut
// so that the schedule and the records fit the scratch array (no split when fewer than
// one record per workgroup slot would fit).  Returns false when even the unsplit
// schedule does not fit.
static bool split_cfg_within(const fmlm_attn_params& p, const Launch& L, int64_t cap, SplitCfg& sc) {
  sc = split_cfg(p, L);
  auto fits = [&](int rec_cap) {
    SplitCfg t = sc;
    t.rec_cap = rec_cap;
    return sched_layout(p, L.bq, t, L.hpack).bytes <= cap;
  };
  if (fits(sc.rec_cap)) return true;
  // the layout grows with the record count: the largest count in [slots, rec_cap) that fits
  int lo = sc.slots, hi = sc.rec_cap - 1;
  if (sc.rec_cap > 0 && lo <= hi && fits(lo)) {
    while (lo < hi) {
      const int mid = lo + (hi - lo + 1) / 2;
      if (fits(mid))
        lo = mid;
      else
        hi = mid - 1;
    }
    sc.rec_cap = lo;
    return true;
  }
  sc.rec_cap = 0;
  return fits(0);
}

}  // namespace fmlm

using namespace fmlm;

extern "C" int fmlm_attn_schedule(const fmlm_attn_params* pp, void* schedule,
                                  int64_t schedule_bytes, void* stream) {
  if (!pp || !schedule || !pp->cu_seqlens_q || pp->B < 1) return FMLM_E_ARG;
  Launch L;
  const int rc = pick_launch(*pp, L);
  if (rc) return rc;
  if (schedule_bytes < workspace_for(*pp, L)) return FMLM_E_WORKSPACE;
  return launch_schedule(*pp, L, split_cfg(*pp, L), (char*)schedule, (hipStream_t)stream);
}

extern "C" int fmlm_attn_params_size(void) { return (int)sizeof(fmlm_attn_params); }

extern "C" int64_t fmlm_attn_workspace_bytes(const fmlm_attn_params* p) {
  if (!p) return FMLM_E_ARG;
  Launch L;
  const int rc = pick_launch(*p, L);
  if (rc) return rc;
  return workspace_for(*p, L);
}

extern "C" int fmlm_attn_fwd(const fmlm_attn_params* pp, void* stream) {
  if (!pp) return FMLM_E_ARG;
  const fmlm_attn_params& p = *pp;
  int rc = check_params(p);
  if (rc) return rc;
  Launch L;
  rc = pick_launch(p, L);
  if (rc) return rc;
  if (p.B == 0 || p.H == 0) return 0;
  const int64_t need = workspace_for(p, L);
  if (need > 0 && !p.schedule && (!p.workspace || p.workspace_bytes < need)) return FMLM_E_WORKSPACE;
  char* sched = (char*)(p.schedule ? p.schedule : p.workspace);
  return launch_attention(p, L, split_cfg(p, L), sched, !p.schedule, (hipStream_t)stream);
}

extern "C" int fmlm_attn_fwd_noalloc(const fmlm_attn_params* pp, void* stream) {
  if (!pp) return FMLM_E_ARG;
  const fmlm_attn_params& p = *pp;
  int rc = check_params(p);
  if (rc) return rc;
  Launch L;
  rc = pick_launch(p, L);
  if (rc) return rc;
  if (p.B == 0 || p.H == 0) return 0;
  SplitCfg sc;
  char* sched = nullptr;
  if (p.cu_seqlens_q) {
    if (!split_cfg_within(p, L, kNoAllocScratchBytes, sc)) return FMLM_E_WORKSPACE;
    rc = scratch_on_current_device(&sched);
    if (rc) return rc;
  }
  // the schedule is always rebuilt: the array holds whatever the previous call left
  return launch_attention(p, L, sc, sched, true, (hipStream_t)stream);
}
