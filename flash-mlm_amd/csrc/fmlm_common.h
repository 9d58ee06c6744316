// Shared device/host helpers for the gfx950 flash-mlm kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flash_mlm_hip.h"

#define FMLM_DEV __device__ __forceinline__

namespace fmlm {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

inline int elem_size(int dtype) {
  switch (dtype) {
    case FMLM_DTYPE_BF16:
    case FMLM_DTYPE_F16:
      return 2;
    case FMLM_DTYPE_F32:
      return 4;
    default:
      return 0;
  }
}

// Element i of a metadata array (sequence offsets, context indices, unit tables) that no
// kernel writes while it reads it.  The read goes through the constant address space, so a
// wave-uniform index becomes a scalar load: it waits on the scalar counter, not on the
// vector-memory counter, and so never waits for the direct tile loads in flight.
typedef const __attribute__((address_space(4))) int32_t cint32_t;
FMLM_DEV int ldc(const int32_t* a, int i) { return ((cint32_t*)(uintptr_t)a)[i]; }

// Start of sequence b in packed token space.
FMLM_DEV int seq_start(const int32_t* cu, int b, int N) { return cu ? ldc(cu, b) : b * N; }

// Index of the sequence whose packed token range [cu[s], cu[s+1]) holds token j
// (cu non-decreasing, 0 <= j < cu[B]).  Empty sequences are skipped because
// the search returns the last s with cu[s] <= j.
FMLM_DEV int find_seq(const int32_t* cu, int B, int j) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (ldc(cu, mid) <= j)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// ---- per-sequence ranges of an attention call
struct SeqInfo {
  int q0, len;       // packed start and clamped length of sequence b
  int ctx, mainlen;  // context keys and main keys it attends to
};

// context batch of sequence b: ctx_index[b] (clamped) when given, else b for a
// full-batch context and 0 for a shared one
FMLM_DEV int ctx_batch_of(const fmlm_attn_params& p, int b) {
  if (p.ctx_index) return min(max(ldc(p.ctx_index, b), 0), max(p.ctx_batch - 1, 0));
  return p.ctx_batch > 1 ? b : 0;
}

// context rows [c0, c1) of context batch cb (contiguous context), or (0, n) of a paged one
FMLM_DEV void ctx_range(const fmlm_attn_params& p, int cb, int& c0, int& c1) {
  c0 = 0;
  c1 = p.ctx_len;
  if (p.cu_seqlens_kv) {
    if (p.ctx_block_table) {
      c1 = ldc(p.cu_seqlens_kv, cb + 1) - ldc(p.cu_seqlens_kv, cb);
    } else {
      c0 = min(max(ldc(p.cu_seqlens_kv, cb), 0), p.ctx_rows);
      c1 = min(max(ldc(p.cu_seqlens_kv, cb + 1), c0), p.ctx_rows);
    }
  }
  if (p.ctx_block_table) c1 = min(max(c1, 0), p.ctx_pages_per_batch * FMLM_PAGE_ROWS);
}

FMLM_DEV SeqInfo seq_info(const fmlm_attn_params& p, int b) {
  const int32_t* cu = p.cu_seqlens_q;
  SeqInfo s;
  s.q0 = seq_start(cu, b, p.N);
  int L = p.N;
  if (cu) {
    L = ldc(cu, b + 1) - s.q0;
    if (p.N > 0) L = min(L, p.N);
    L = max(min(L, p.total_q - s.q0), 0);
  }
  s.len = L;
  s.ctx = 0;
  if (!(p.flags & FMLM_FLAG_PREFILL)) {
    int c0, c1;
    ctx_range(p, ctx_batch_of(p, b), c0, c1);
    s.ctx = max(c1 - c0, 0);
  }
  s.mainlen = ((p.flags & FMLM_FLAG_CAUSAL_SEQ) && cu) ? s.q0 + L : L;
  return s;
}

FMLM_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// ---- MFMA 16x16x32 and the transposed LDS read
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

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define FMLM_LDS __attribute__((address_space(3)))

// ds_read_b64_tr_b16: within each group of 16 lanes, lane j supplies the address of
// four consecutive 16-bit elements M[j][0..3]; lane i receives M[4e + i/4][i%4], e=0..3.
FMLM_DEV s16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((FMLM_LDS s16x4*)(p));
}
// the same from an LDS byte address
FMLM_DEV s16x4 lds_read_tr16_at(uint32_t a) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((FMLM_LDS s16x4*)(uintptr_t)a);
}

// 16-byte chunk swizzles of a row-major LDS tile of head dim D: logical chunk c of row r
// sits in physical chunk c ^ swz(r), swz depending on r % 16 only.  Two read shapes use
// the tiles: b128 row fragments (lane (l16 + 16g) reads chunk 4b + g of row l16) and tr16
// column fragments (lane (l16 + 16g) reads 8 bytes of row 4g + l16/4).  gfx950's LDS has
// 64 banks of 4 bytes; a tr16 (or b64) read serves 32 consecutive lanes per cycle, so it
// is conflict free when the 8 rows of those lanes put their 32-byte column block in 8
// different bank groups: bits 1-3 of swz a bijection on rows 0-7 and on rows 8-15.  The
// b128 lane grouping is not documented; measured read patterns (SQ_LDS_BANK_CONFLICT of
// one pattern per launch) fit several models of 8-lane groups, and the D >= 128 swizzle
// below is conflict free for both read shapes under every model that fits and in
// measurement at row pitches of 256, 512 and 1024 bytes (an XOR-linear map of the 4 row
// bits: 1 -> 2, 2 -> 4, 4 -> 9, 8 -> 12).  The former D >= 128 swizzle,
// ((r & 7) << 1) | ((r >> 3) & 1), served tr16 reads but cost b128 reads two cycles per
// 16 lanes, and r & 15 the reverse.
//   kv_swz: conflict free for b128 and tr16 reads at every D;
//   k_swz:  the swizzle of tiles read by b128 only (the forward's K tiles).
template <int D>
FMLM_DEV int kv_swz(int r) {
  if constexpr (D >= 128) return ((r & 3) << 1) ^ (((r >> 2) & 1) * 9) ^ (((r >> 3) & 1) * 12);
  else if constexpr (D == 64) return r & 7;
  else if constexpr (D == 32) return (r >> 1) & 3;
  else return (r >> 3) & 1;
}
template <int D>
FMLM_DEV int k_swz(int r) {
  if constexpr (D >= 128) return r & 15;
  else return kv_swz<D>(r);
}

// An empty asm that claims to rewrite x: arithmetic producing x stays before this point
// and arithmetic consuming it stays after, in the order of the surrounding side effects.
template <typename X>
FMLM_DEV void pin(X& x) { asm volatile("" : "+v"(x)); }

// two elements of the input type (a packed 32-bit pair)
template <typename T>
struct Pair;
template <>
struct Pair<bf16> {
  typedef __bf16 type __attribute__((ext_vector_type(2)));
};
template <>
struct Pair<f16> {
  typedef _Float16 type __attribute__((ext_vector_type(2)));
};
typedef float f32x2 __attribute__((ext_vector_type(2)));

FMLM_DEV float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max over lanes l, l^16, l^32, l^48: permlane16/32_swap(x, x) return {x[l], x[l^16]}
// resp. {x[l], x[l^32]} in some order
FMLM_DEV float lane_max_xor16_32(float x) {
  const int xi = __builtin_bit_cast(int, x);
  const auto a = __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
  x = vmax(__builtin_bit_cast(float, (int)a[0]), __builtin_bit_cast(float, (int)a[1]));
  const int yi = __builtin_bit_cast(int, x);
  const auto b = __builtin_amdgcn_permlane32_swap(yi, yi, false, false);
  return vmax(__builtin_bit_cast(float, (int)b[0]), __builtin_bit_cast(float, (int)b[1]));
}

FMLM_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const FMLM_LDS char*)p;
}

FMLM_DEV const char* uniform_ptr(const char* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const char*)(((uint64_t)hi << 32) | lo);
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 64 lanes x 16 bytes from base + off (per lane) to LDS [lds, lds + 1024), lane l at
// lds + 16 l.  base and lds are wave-uniform.
FMLM_DEV void dma16_sbase(const char* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(off), "s"(base), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

}  // namespace fmlm
