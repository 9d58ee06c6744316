// Indexing kernels of the packed MLM path: pack metadata, pack and unpack.
//
// These replace the torch-op chains of the reference host layer:
//   build_pack_metadata / _build_query_tile_map_from_cu_seqlens  host_utils.py:27-107
//   _pack_flatten_for_kernel_into (+ its permute().contiguous())  host_utils.py:397-420
//   unpack_from_kernel (zeros + index_copy_ + permute)           host_utils.py:587-615
// Each is one pass over HBM: pack reads every valid padded row once and writes
// every packed row once; unpack writes every padded row once (zeros included).
#include "fmlm_common.h"

#include <algorithm>

namespace fmlm {

// ---------------------------------------------------------------------------
// Pack metadata, step 1: one workgroup scans the lengths.
//   cu[0] = 0, cu[i+1] = cu[i] + L_i                         (host_utils.py:49-50)
//   tiles_i = ceil(L_i / block_n), tp = exclusive scan       (host_utils.py:84-96)
// Lengths outside [0, N] are counted (host_utils.py:42-43) and treated as 0 in
// the scan so every later index stays in bounds.
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 1024;

template <typename LT>
__global__ __launch_bounds__(kScanThreads) void metadata_scan_kernel(
    const LT* __restrict__ lengths, int B, int N, int block_n, int32_t* __restrict__ lengths_i32,
    int32_t* __restrict__ aux) {
  __shared__ int s_len[kScanThreads];
  __shared__ int s_til[kScanThreads];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  int32_t* cu = aux;
  int32_t* summary = aux + B + 1;
  int32_t* tp = aux + B + 5;
  if (tid == 0) {
    s_bad = 0;
    cu[0] = 0;
    tp[0] = 0;
  }
  int carry_len = 0, carry_til = 0;
  __syncthreads();
  for (int base = 0; base < B; base += kScanThreads) {
    const int i = base + tid;
    int len = 0;
    if (i < B) {
      const LT raw = lengths[i];
      const bool ok = raw >= 0 && raw <= (LT)N;
      lengths_i32[i] = (int32_t)raw;
      if (!ok) atomicAdd(&s_bad, 1);
      len = ok ? (int)raw : 0;
    }
    s_len[tid] = len;
    s_til[tid] = (len + block_n - 1) / block_n;
    __syncthreads();
    // Hillis-Steele inclusive scan over the chunk.
    for (int off = 1; off < kScanThreads; off <<= 1) {
      int a = 0, t = 0;
      if (tid >= off) {
        a = s_len[tid - off];
        t = s_til[tid - off];
      }
      __syncthreads();
      s_len[tid] += a;
      s_til[tid] += t;
      __syncthreads();
    }
    if (i < B) {
      cu[i + 1] = carry_len + s_len[tid];
      tp[i + 1] = carry_til + s_til[tid];
    }
    carry_len += s_len[kScanThreads - 1];
    carry_til += s_til[kScanThreads - 1];
    __syncthreads();
  }
  if (tid == 0) {
    summary[0] = carry_len;  // total_tokens
    summary[1] = carry_til;  // n_tiles
    summary[2] = s_bad;      // lengths outside [0, N]
    summary[3] = 0;
  }
}

// Pack metadata, step 2: every (b, t < L_b) writes its packed token index and
// every (b, j < tiles_b) its tile entry (host_utils.py:52-55, 97-106).
__global__ __launch_bounds__(256) void metadata_fill_kernel(
    const int32_t* __restrict__ lengths_i32, const int32_t* __restrict__ aux, int B, int N,
    int block_n, int chunks_per_seq, int64_t* __restrict__ token_indices,
    int32_t* __restrict__ batch_ids, int32_t* __restrict__ tile_starts) {
  if (aux[B + 3] != 0) return;  // invalid lengths: the host raises
  const int b = blockIdx.x / chunks_per_seq;
  const int t = (blockIdx.x % chunks_per_seq) * 256 + threadIdx.x;
  const int len = lengths_i32[b];
  const int start = aux[b];
  if (t < len) token_indices[start + t] = (int64_t)b * N + t;
  const int tiles = (len + block_n - 1) / block_n;
  if (t < tiles) {
    const int slot = aux[B + 5 + b] + t;
    batch_ids[slot] = b;
    tile_starts[slot] = start + t * block_n;
  }
}

// Tile map from cu_seqlens (host_utils.py:74-107): one workgroup scans the tile
// counts and writes (b, cu[b] + j*block_n) for every tile, capped at capacity.
__global__ __launch_bounds__(kScanThreads) void tile_map_kernel(const int32_t* __restrict__ cu,
                                                                int B, int block_n, int capacity,
                                                                int32_t* __restrict__ batch_ids,
                                                                int32_t* __restrict__ tile_starts,
                                                                int32_t* __restrict__ count) {
  __shared__ int s_til[kScanThreads];
  const int tid = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < B; base += kScanThreads) {
    const int b = base + tid;
    int tiles = 0, start = 0;
    if (b < B) {
      start = cu[b];
      const int len = cu[b + 1] - start;
      tiles = len > 0 ? (len + block_n - 1) / block_n : 0;
    }
    s_til[tid] = tiles;
    __syncthreads();
    for (int off = 1; off < kScanThreads; off <<= 1) {
      const int t = tid >= off ? s_til[tid - off] : 0;
      __syncthreads();
      s_til[tid] += t;
      __syncthreads();
    }
    const int first = carry + s_til[tid] - tiles;
    for (int j = 0; j < tiles && first + j < capacity; ++j) {
      batch_ids[first + j] = b;
      tile_starts[first + j] = start + j * block_n;
    }
    carry += s_til[kScanThreads - 1];
    __syncthreads();
  }
  if (tid == 0) *count = carry;
}

// ---------------------------------------------------------------------------
// Pack: one thread per VB-byte chunk of a packed row.
// ---------------------------------------------------------------------------
template <int VB>
struct VecOf;
template <>
struct VecOf<16> {
  typedef u32x4 type;
};
template <>
struct VecOf<8> {
  typedef u32x2 type;
};
template <>
struct VecOf<4> {
  typedef uint32_t type;
};
template <>
struct VecOf<2> {
  typedef uint16_t type;
};
template <>
struct VecOf<1> {
  typedef uint8_t type;
};

struct PackArgs {
  fmlm_pack_tensor t[3];
};

// ---------------------------------------------------------------------------
// Span copies.  Pack, unpack and the KV append each move, per (sequence or segment,
// head), one contiguous run of rows to another contiguous run, with zero rows around.
// A workgroup takes a window of kWin bytes of one such destination span: every thread
// moves kPer vectors of VB bytes, issuing all its loads before its stores, and the
// threads of one vector index cover kSpanThreads * VB consecutive bytes.  Pack and the KV
// append size their grids to the average sequence (batch) length, and longer ones loop
// over further windows: a grid sized to the longest left many workgroups with nothing to
// copy.  Their windows are smaller than the other span kernels' (kPackPer, kAppendPer
// vectors per thread), which balances that loop.  Measured against kPer-vector windows:
// pack with an N-sized grid -> average-sized with two vectors, config 3 0.67 -> 0.78 of
// HBM peak, config 5 0.67 -> 0.69, config 4 0.33 -> 0.42; append with one vector, config 3
// 0.69 -> 0.75, config 5 0.63 -> 0.69.  Non-temporal stores were slower in every kernel.
// ---------------------------------------------------------------------------
constexpr int kSpanThreads = 256;
constexpr int kPer = 4;
constexpr int kAppendPer = 1;
constexpr int kPackPer = 2;

template <int VB, int PER = kPer>
struct Span {
  typedef typename VecOf<VB>::type V;
  static constexpr int64_t kWin = (int64_t)kSpanThreads * PER * VB;
};

// Bytes [w0, w0 + kWin) of a destination span of `len` bytes: offsets below `cpy` come from
// src at the same offset, the rest are zero.  src_row_bytes / src_pitch (bytes) read a
// strided source: offset o is row o / src_row_bytes, column o % src_row_bytes, at
// row * src_pitch + column (src_pitch == src_row_bytes: contiguous).
template <int VB, bool STRIDED, int PER = kPer>
FMLM_DEV void span_window(const char* __restrict__ src, char* __restrict__ dst, int64_t w0, int64_t len,
                          int64_t cpy, uint32_t src_row_bytes, int64_t src_pitch) {
  typedef typename Span<VB>::V V;
  V v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t o = w0 + ((int64_t)i * kSpanThreads + threadIdx.x) * VB;
    v[i] = V{};
    if (o < cpy) {
      int64_t so = o;
      if constexpr (STRIDED) {
        const uint32_t r = (uint32_t)o / src_row_bytes;
        so = (int64_t)r * src_pitch + ((uint32_t)o - r * src_row_bytes);
      }
      v[i] = *(const V*)(src + so);
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t o = w0 + ((int64_t)i * kSpanThreads + threadIdx.x) * VB;
    if (o < len) *(V*)(dst + o) = v[i];
  }
}

// ---------------------------------------------------------------------------
// Pack: grid (window, tensor*heads, sequence).  Sequence b's rows p < min(L_b, N) of head
// h go to dst rows h*T_pad + cu[b] + p (clamped to [0, T)); the last grid slice (z = B)
// zero-fills the rows of [0, T_pad) outside [cu[0], cu[B]) (the packed tail [T, T_pad) for
// consistent metadata).  Without cu_seqlens, sequence b covers rows [b*N, (b+1)*N).
// Source rows are contiguous when s_sn is the row length (STRIDED otherwise).
// ---------------------------------------------------------------------------
template <int VB, bool STRIDED>
__global__ __launch_bounds__(kSpanThreads) void pack_kernel(PackArgs args, int n_tensors, int hmax, int esz,
                                                            int B, int N, int D,
                                                            const int32_t* __restrict__ cu, int T,
                                                            int T_pad) {
  const int ti = blockIdx.y / hmax, h = blockIdx.y % hmax;
  if (ti >= n_tensors) return;
  const fmlm_pack_tensor& tt = args.t[ti];
  if (h >= tt.heads) return;
  const int64_t row_bytes = (int64_t)D * esz;
  char* const dst = (char*)tt.dst + (int64_t)h * T_pad * row_bytes;
  const int b = blockIdx.z;
  if (b < B) {
    const int start = cu ? cu[b] : b * N;
    int len = min(cu ? cu[b + 1] - start : N, N);
    if (start < 0 || start >= T) return;
    len = min(len, T - start);
    const int64_t bytes = (int64_t)max(len, 0) * row_bytes;
    const char* src = (const char*)tt.src + ((int64_t)b * tt.s_sb + (int64_t)h * tt.s_sh) * esz;
    typedef Span<VB, kPackPer> W;
    for (int64_t w0 = (int64_t)blockIdx.x * W::kWin; w0 < bytes; w0 += (int64_t)gridDim.x * W::kWin)
      span_window<VB, STRIDED, kPackPer>(src, dst + (int64_t)start * row_bytes, w0, bytes, bytes,
                                         (uint32_t)row_bytes, tt.s_sn * esz);
  } else {  // zero rows outside [c0, c1): the spans [0, c0) and [c1, T_pad)
    const int c0 = cu ? min(max(cu[0], 0), T) : 0;
    const int c1 = cu ? min(max(cu[B], c0), T) : T;
    const int64_t lo = (int64_t)c0 * row_bytes, hi = (int64_t)(T_pad - c1) * row_bytes;
    // windows [0, nlo) cover the span [0, c0), the rest the span [c1, T_pad) from its own
    // offset 0 (a shared byte range would skip the first bytes of the second span when
    // lo is not a whole number of windows)
    constexpr int64_t kWin = Span<VB>::kWin;
    const int64_t nlo = (lo + kWin - 1) / kWin, nwin = nlo + (hi + kWin - 1) / kWin;
    for (int64_t i = blockIdx.x; i < nwin; i += gridDim.x) {
      if (i < nlo)
        span_window<VB, false>(nullptr, dst, i * kWin, lo, 0, 1u, 0);
      else
        span_window<VB, false>(nullptr, dst + (int64_t)c1 * row_bytes, (i - nlo) * kWin, hi, 0, 1u, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Unpack: block (TX chunk lanes x TY rows) over grid (row block of N, head, sequence):
// dst row (b, h, n) = packed row h*p_sh/D + cu[b] + n for n < L_b, zeros otherwise.  (One
// 16-byte chunk per thread measured faster here than the span windows pack uses.)
// ---------------------------------------------------------------------------
template <int VB>
__global__ __launch_bounds__(256) void unpack_kernel(const char* __restrict__ packed, int64_t p_sh,
                                                     char* __restrict__ dst, int B, int H, int N,
                                                     int D, int esz,
                                                     const int32_t* __restrict__ cu) {
  typedef typename VecOf<VB>::type V;
  const int cpr = D * esz / VB;
  const int64_t row_bytes = (int64_t)D * esz;
  const int h = blockIdx.y, b = blockIdx.z;
  const int start = cu[b];
  const int len = cu[b + 1] - start;
  const int n = blockIdx.x * blockDim.y + threadIdx.y;
  if (n >= N) return;
  char* const out = dst + (((int64_t)b * H + h) * N + n) * row_bytes;
  if (n < len) {
    const char* in = packed + ((int64_t)h * p_sh + (int64_t)(start + n) * D) * esz;
    for (int c = threadIdx.x; c < cpr; c += blockDim.x)
      *(V*)(out + (int64_t)c * VB) = *(const V*)(in + (int64_t)c * VB);
  } else {
    for (int c = threadIdx.x; c < cpr; c += blockDim.x) *(V*)(out + (int64_t)c * VB) = V{};
  }
}

// Block shape for a row-copy kernel: TX lanes across a row's chunks, TY rows.
static dim3 row_block(int cpr) {
  const int tx = cpr < 256 ? cpr : 256;
  return dim3(tx, 256 / tx);
}

// ---------------------------------------------------------------------------
// Segment copy (KV append): grid (windows, head, segment).  Segment c of head h: rows
// [src_cu[c], src_cu[c+1]) of src (head stride src_sh elements) go to rows
// [dst_start[c], dst_start[c] + len) of dst (head stride dst_sh).  Lengths and starts are
// clamped to the row counts of src and dst, so inconsistent offsets cannot address
// outside either tensor.  The windows stride over the segment, so the grid does not
// depend on segment lengths the host has not read.  A null src writes zero rows (src_rows
// then only bounds the segment offsets).
// ---------------------------------------------------------------------------
template <int VB>
__global__ __launch_bounds__(kSpanThreads) void segment_copy_kernel(const char* __restrict__ src, int64_t src_sh,
                                                                    int src_rows, const int32_t* __restrict__ src_cu,
                                                                    char* __restrict__ dst, int64_t dst_sh,
                                                                    int dst_rows, const int32_t* __restrict__ dst_start,
                                                                    int D, int esz) {
  const int h = blockIdx.y, c = blockIdx.z;
  const int s0 = min(max(src_cu[c], 0), src_rows);
  const int d0 = min(max(dst_start[c], 0), dst_rows);
  const int len = max(min(min(src_cu[c + 1] - s0, src_rows - s0), dst_rows - d0), 0);
  const int64_t row_bytes = (int64_t)D * esz;
  const int64_t bytes = (int64_t)len * row_bytes;
  const char* const sbase = src ? src + ((int64_t)h * src_sh + (int64_t)s0 * D) * esz : nullptr;
  char* const dbase = dst + ((int64_t)h * dst_sh + (int64_t)d0 * D) * esz;
  for (int64_t w0 = (int64_t)blockIdx.x * Span<VB>::kWin; w0 < bytes; w0 += (int64_t)gridDim.x * Span<VB>::kWin)
    span_window<VB, false>(sbase, dbase, w0, bytes, src ? bytes : 0, 1u, 0);
}

// ---------------------------------------------------------------------------
// KV append in one launch: grid (windows, tensor*heads, batch + 1).  Batch c of head h of
// the merged entry (rows [o_c, o_{c+1}) with o = cu_old + cu_new) is the old rows
// [cu_old[c], cu_old[c+1]) followed by the new rows [cu_new[c], cu_new[c+1]); the last
// grid slice zero-fills rows [o_C, t_old + t_new) (the entry's tail, like a prefilled
// entry's padding rows).  Offsets are clamped to the buffers' rows; workgroup (0, 0, 0)
// also writes cu_out = o.
// ---------------------------------------------------------------------------
struct AppendArgs {
  fmlm_append_tensor t[2];
};

template <int VB>
__global__ __launch_bounds__(kSpanThreads) void kv_append_kernel(AppendArgs args, int n_tensors, int H, int D,
                                                                 int esz, int C, int t_old, int t_new,
                                                                 const int32_t* __restrict__ cu_old,
                                                                 const int32_t* __restrict__ cu_new,
                                                                 int32_t* __restrict__ cu_out) {
  typedef typename Span<VB>::V V;
  const int c = blockIdx.z;
  if (cu_out && blockIdx.x == 0 && blockIdx.y == 0 && c == 0)
    for (int i = threadIdx.x; i <= C; i += blockDim.x) cu_out[i] = cu_old[i] + cu_new[i];
  const int ti = blockIdx.y / H, h = blockIdx.y % H;
  if (ti >= n_tensors) return;
  const fmlm_append_tensor& tt = args.t[ti];
  const int64_t row_bytes = (int64_t)D * esz;
  const int rows = t_old + t_new;
  char* const out = (char*)tt.out + (int64_t)h * rows * row_bytes;
  auto clampr = [](int x, int hi) { return min(max(x, 0), hi); };
  if (c < C) {
    const int a0 = clampr(cu_old[c], t_old), a1 = clampr(cu_old[c + 1], t_old);
    const int b0 = clampr(cu_new[c], t_new), b1 = clampr(cu_new[c + 1], t_new);
    const int na = max(a1 - a0, 0), nb = max(b1 - b0, 0);
    const int o0 = clampr(cu_old[c] + cu_new[c], rows);
    const int64_t old_bytes = (int64_t)min(na, rows - o0) * row_bytes;
    const int64_t bytes = (int64_t)min(na + nb, rows - o0) * row_bytes;
    const char* const sa = (const char*)tt.old + ((int64_t)h * t_old + a0) * row_bytes;
    const char* const sb = (const char*)tt.add + ((int64_t)h * t_new + b0) * row_bytes;
    char* const d = out + (int64_t)o0 * row_bytes;
    typedef Span<VB, kAppendPer> W;
    for (int64_t w0 = (int64_t)blockIdx.x * W::kWin; w0 < bytes; w0 += (int64_t)gridDim.x * W::kWin) {
      V v[kAppendPer];
#pragma unroll
      for (int i = 0; i < kAppendPer; ++i) {
        const int64_t o = w0 + ((int64_t)i * kSpanThreads + threadIdx.x) * VB;
        v[i] = V{};
        if (o < old_bytes)
          v[i] = *(const V*)(sa + o);
        else if (o < bytes)
          v[i] = *(const V*)(sb + (o - old_bytes));
      }
#pragma unroll
      for (int i = 0; i < kAppendPer; ++i) {
        const int64_t o = w0 + ((int64_t)i * kSpanThreads + threadIdx.x) * VB;
        if (o < bytes) *(V*)(d + o) = v[i];
      }
    }
  } else {  // the tail rows of the head
    const int o_end = clampr(cu_old[C] + cu_new[C], rows);
    const int64_t bytes = (int64_t)(rows - o_end) * row_bytes;
    for (int64_t w0 = (int64_t)blockIdx.x * Span<VB>::kWin; w0 < bytes; w0 += (int64_t)gridDim.x * Span<VB>::kWin)
      span_window<VB, false>(nullptr, out + (int64_t)o_end * row_bytes, w0, bytes, 0, 1u, 0);
  }
}

// Widest vector width (bytes) that divides the row size and every address.
static int pick_vec(int64_t row_bytes, std::initializer_list<uint64_t> addrs_bytes) {
  for (int vb : {16, 8, 4, 2, 1}) {
    if (row_bytes % vb) continue;
    bool ok = true;
    for (uint64_t a : addrs_bytes) ok = ok && (a % vb == 0);
    if (ok) return vb;
  }
  return 0;
}

}  // namespace fmlm

using namespace fmlm;

extern "C" int fmlm_abi_version(void) { return FMLM_ABI_VERSION; }
extern "C" int fmlm_pack_tensor_size(void) { return (int)sizeof(fmlm_pack_tensor); }

extern "C" int fmlm_pack_metadata(const void* lengths, int32_t lengths_is_i64, int32_t B,
                                  int32_t N, int32_t block_n, int32_t* lengths_i32, int32_t* aux,
                                  int64_t* token_indices, int32_t* batch_ids,
                                  int32_t* tile_starts, void* stream) {
  if (B < 0 || N < 0 || block_n < 1 || !aux) return FMLM_E_ARG;
  if (B > 0 && (!lengths || !lengths_i32)) return FMLM_E_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (lengths_is_i64)
    hipLaunchKernelGGL(metadata_scan_kernel<int64_t>, dim3(1), dim3(kScanThreads), 0, s,
                       (const int64_t*)lengths, B, N, block_n, lengths_i32, aux);
  else
    hipLaunchKernelGGL(metadata_scan_kernel<int32_t>, dim3(1), dim3(kScanThreads), 0, s,
                       (const int32_t*)lengths, B, N, block_n, lengths_i32, aux);
  int rc = launch_status();
  if (rc || B == 0 || N == 0) return rc;
  if (!token_indices || !batch_ids || !tile_starts) return FMLM_E_ARG;
  const int chunks = (N + 255) / 256;
  const int64_t blocks = (int64_t)B * chunks;
  if (blocks > 0x7fffffff) return FMLM_E_ARG;
  hipLaunchKernelGGL(metadata_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, s, lengths_i32,
                     aux, B, N, block_n, chunks, token_indices, batch_ids, tile_starts);
  return launch_status();
}

extern "C" int fmlm_tile_map(const int32_t* cu_seqlens, int32_t B, int32_t block_n,
                             int32_t capacity, int32_t* batch_ids, int32_t* tile_starts,
                             int32_t* count, void* stream) {
  if (B < 0 || block_n < 1 || capacity < 0 || !count) return FMLM_E_ARG;
  if (B > 0 && !cu_seqlens) return FMLM_E_ARG;
  if (capacity > 0 && (!batch_ids || !tile_starts)) return FMLM_E_ARG;
  hipLaunchKernelGGL(tile_map_kernel, dim3(1), dim3(kScanThreads), 0, (hipStream_t)stream,
                     cu_seqlens, B, block_n, capacity, batch_ids, tile_starts, count);
  return launch_status();
}

static bool valid_elem_bytes(int e) { return e == 1 || e == 2 || e == 4 || e == 8; }

extern "C" int fmlm_pack(const fmlm_pack_tensor* tensors, int32_t n_tensors, int32_t elem_bytes,
                         int32_t B, int32_t N, int32_t D, const int32_t* cu_seqlens, int32_t T,
                         int32_t T_pad, void* stream) {
  const int esz = elem_bytes;
  if (!valid_elem_bytes(esz)) return FMLM_E_DTYPE;
  if (!tensors || n_tensors < 1 || n_tensors > 3 || B < 0 || N < 0 || D < 1 || T < 0 ||
      T_pad < T)
    return FMLM_E_ARG;
  if (!cu_seqlens && T != B * N) return FMLM_E_ARG;
  PackArgs args = {};
  int vb = 16;
  for (int i = 0; i < n_tensors; ++i) {
    const fmlm_pack_tensor& t = tensors[i];
    if (t.heads < 1 || !t.dst || (T > 0 && !t.src)) return FMLM_E_ARG;
    args.t[i] = t;
    const int v = pick_vec((int64_t)D * esz,
                           {(uint64_t)t.src, (uint64_t)t.dst, (uint64_t)(t.s_sb * esz),
                            (uint64_t)(t.s_sh * esz), (uint64_t)(t.s_sn * esz)});
    if (!v) return FMLM_E_ALIGN;
    vb = v < vb ? v : vb;
  }
  if (T_pad == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  int hmax = 0;
  for (int i = 0; i < n_tensors; ++i) hmax = tensors[i].heads > hmax ? tensors[i].heads : hmax;
  // windows per sequence span at the average sequence length (longer sequences loop over
  // further windows); the zero slice strides over its rows
  const int64_t win = (int64_t)kSpanThreads * kPackPer * vb;
  const int64_t avg = B > 0 ? std::min<int64_t>(N, ((int64_t)T + B - 1) / B) : N;
  const int64_t gx = std::max<int64_t>(1, ((int64_t)(avg > 0 ? avg : 1) * D * esz + win - 1) / win);
  if ((int64_t)hmax * n_tensors > 65535 || B + 1 > 65535 || gx > (1 << 30)) return FMLM_E_ARG;
  const dim3 grid((unsigned)gx, hmax * n_tensors, B + 1);
  // source rows are contiguous when every tensor's row stride is the row length
  bool strided = false;
  for (int i = 0; i < n_tensors; ++i) strided = strided || tensors[i].s_sn != D;
#define FMLM_PACK_CASE(VB)                                                                              \
  case VB:                                                                                              \
    if (strided)                                                                                        \
      hipLaunchKernelGGL((pack_kernel<VB, true>), grid, dim3(kSpanThreads), 0, s, args, n_tensors, hmax, \
                         esz, B, N, D, cu_seqlens, T, T_pad);                                           \
    else                                                                                                \
      hipLaunchKernelGGL((pack_kernel<VB, false>), grid, dim3(kSpanThreads), 0, s, args, n_tensors,     \
                         hmax, esz, B, N, D, cu_seqlens, T, T_pad);                                     \
    break;
  switch (vb) {
    FMLM_PACK_CASE(16)
    FMLM_PACK_CASE(8)
    FMLM_PACK_CASE(4)
    FMLM_PACK_CASE(2)
    FMLM_PACK_CASE(1)
  }
#undef FMLM_PACK_CASE
  return launch_status();
}

extern "C" int fmlm_unpack(int32_t elem_bytes, const void* packed, int64_t p_sh, void* dst,
                           int32_t B, int32_t H, int32_t N, int32_t D, const int32_t* cu_seqlens,
                           void* stream) {
  const int esz = elem_bytes;
  if (!valid_elem_bytes(esz)) return FMLM_E_DTYPE;
  if (B < 0 || H < 0 || N < 0 || D < 1 || p_sh < 0 || !cu_seqlens) return FMLM_E_ARG;
  const int64_t rows = (int64_t)B * H * N;
  if (rows == 0) return 0;
  if (!dst) return FMLM_E_ARG;
  const int vb = pick_vec((int64_t)D * esz,
                          {(uint64_t)packed, (uint64_t)dst, (uint64_t)(p_sh * esz)});
  if (!vb) return FMLM_E_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const dim3 blk = row_block((int)((int64_t)D * esz / vb));
  const int64_t gx = ((int64_t)N + blk.y - 1) / blk.y;
  if (H > 65535 || B > 65535 || gx > (1 << 30)) return FMLM_E_ARG;
  const dim3 grid((unsigned)gx, H, B);
  const char* pk = (const char*)packed;
  char* out = (char*)dst;
#define FMLM_UNPACK_CASE(VB)                                                                 \
  case VB:                                                                                   \
    hipLaunchKernelGGL(unpack_kernel<VB>, grid, blk, 0, s, pk, p_sh, out, B, H, N, D, esz, \
                       cu_seqlens);                                                          \
    break;
  switch (vb) {
    FMLM_UNPACK_CASE(16)
    FMLM_UNPACK_CASE(8)
    FMLM_UNPACK_CASE(4)
    FMLM_UNPACK_CASE(2)
    FMLM_UNPACK_CASE(1)
  }
#undef FMLM_UNPACK_CASE
  return launch_status();
}

extern "C" int fmlm_copy_segments(int32_t elem_bytes, const void* src, int64_t src_sh, int32_t src_rows,
                                  const int32_t* src_cu, void* dst, int64_t dst_sh, int32_t dst_rows,
                                  const int32_t* dst_start, int32_t C, int32_t H, int32_t D, void* stream) {
  const int esz = elem_bytes;
  if (!valid_elem_bytes(esz)) return FMLM_E_DTYPE;
  if (C < 0 || H < 0 || D < 1 || src_rows < 0 || dst_rows < 0 || src_sh < 0 || dst_sh < 0) return FMLM_E_ARG;
  if ((int64_t)C * H == 0 || src_rows == 0 || dst_rows == 0) return 0;
  if (!dst || !src_cu || !dst_start) return FMLM_E_ARG;
  if (H > 65535 || C > 65535) return FMLM_E_ARG;
  const int vb = pick_vec((int64_t)D * esz, {(uint64_t)src, (uint64_t)dst, (uint64_t)(src_sh * esz),
                                             (uint64_t)(dst_sh * esz)});
  if (!vb) return FMLM_E_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  // windows per (head, segment) at the average segment length; longer segments are
  // covered by the stride loop
  const int64_t win = (int64_t)kSpanThreads * kPer * vb;
  const int64_t avg = ((int64_t)src_rows + C - 1) / C;
  const int64_t gx = std::max<int64_t>(1, std::min<int64_t>((avg * D * esz + win - 1) / win, 4096));
  const dim3 grid((unsigned)gx, H, C);
  const char* sp = (const char*)src;
  char* dp = (char*)dst;
#define FMLM_SEG_CASE(VB)                                                                                   \
  case VB:                                                                                                  \
    hipLaunchKernelGGL(segment_copy_kernel<VB>, grid, dim3(kSpanThreads), 0, s, sp, src_sh, src_rows, src_cu, \
                       dp, dst_sh, dst_rows, dst_start, D, esz);                                             \
    break;
  switch (vb) {
    FMLM_SEG_CASE(16)
    FMLM_SEG_CASE(8)
    FMLM_SEG_CASE(4)
    FMLM_SEG_CASE(2)
    FMLM_SEG_CASE(1)
  }
#undef FMLM_SEG_CASE
  return launch_status();
}

extern "C" int fmlm_kv_append(const fmlm_append_tensor* tensors, int32_t n_tensors, int32_t elem_bytes, int32_t H,
                              int32_t D, int32_t C, int32_t t_old, int32_t t_new, const int32_t* cu_old,
                              const int32_t* cu_new, int32_t* cu_out, void* stream) {
  const int esz = elem_bytes;
  if (!valid_elem_bytes(esz)) return FMLM_E_DTYPE;
  if (!tensors || n_tensors < 1 || n_tensors > 2 || H < 0 || D < 1 || C < 0 || t_old < 0 || t_new < 0)
    return FMLM_E_ARG;
  const int64_t rows = (int64_t)t_old + t_new;
  if (rows > 0x7fffffff) return FMLM_E_ARG;
  // every launch below reads cu_old[0..C] and cu_new[0..C] (the tail slice reads index C
  // even when C == 0); the only call that launches nothing is the empty one
  const bool launches = (H > 0 && rows > 0) || (cu_out && C > 0);
  if (launches && (!cu_old || !cu_new)) return FMLM_E_ARG;
  if (H == 0 || rows == 0) {  // nothing to move: only the offsets
    if (!cu_out || C == 0) return 0;
    AppendArgs args = {};
    hipLaunchKernelGGL(kv_append_kernel<16>, dim3(1), dim3(kSpanThreads), 0, (hipStream_t)stream, args, 0, 1, D,
                       esz, C, t_old, t_new, cu_old, cu_new, cu_out);
    return launch_status();
  }
  AppendArgs args = {};
  int vb = 16;
  for (int i = 0; i < n_tensors; ++i) {
    const fmlm_append_tensor& t = tensors[i];
    if (!t.out || (t_old > 0 && !t.old) || (t_new > 0 && !t.add)) return FMLM_E_ARG;
    args.t[i] = t;
    const int v = pick_vec((int64_t)D * esz, {(uint64_t)t.old, (uint64_t)t.add, (uint64_t)t.out});
    if (!v) return FMLM_E_ALIGN;
    vb = v < vb ? v : vb;
  }
  if ((int64_t)H * n_tensors > 65535 || C + 1 > 65535) return FMLM_E_ARG;
  // windows per (tensor, head, batch) at the average merged batch length; longer batches
  // are covered by the stride loop
  const int64_t win = (int64_t)kSpanThreads * kAppendPer * vb;
  const int64_t avg = (rows + C) / (C + 1);
  const int64_t gx = std::max<int64_t>(1, std::min<int64_t>((avg * D * esz + win - 1) / win, 4096));
  const dim3 grid((unsigned)gx, H * n_tensors, C + 1);
  hipStream_t s = (hipStream_t)stream;
#define FMLM_APPEND_CASE(VB)                                                                              \
  case VB:                                                                                                \
    hipLaunchKernelGGL(kv_append_kernel<VB>, grid, dim3(kSpanThreads), 0, s, args, n_tensors, H, D, esz, C, \
                       t_old, t_new, cu_old, cu_new, cu_out);                                             \
    break;
  switch (vb) {
    FMLM_APPEND_CASE(16)
    FMLM_APPEND_CASE(8)
    FMLM_APPEND_CASE(4)
    FMLM_APPEND_CASE(2)
    FMLM_APPEND_CASE(1)
  }
#undef FMLM_APPEND_CASE
  return launch_status();
}
