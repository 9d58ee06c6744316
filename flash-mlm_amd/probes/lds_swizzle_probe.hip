// LDS bank-conflict probe for the chunk swizzles of the attention kernels' tiles.
//
// Each launch reads LDS in one fixed per-lane pattern (a 64-entry table of byte
// addresses, all inside a 64 KiB buffer), 4 reads per iteration, ITER iterations, so the
// SQ counters of that dispatch describe the pattern alone.  Patterns: the K-fragment read
// (ds_read_b128: lane (l16 + 16g) reads row l16, logical chunk 4kc + g) and the
// V-fragment read (ds_read_b64_tr_b16: lane (l16 + 16g) reads 8 bytes of row 4g + l16/4,
// logical chunk 2db + (l16 & 3)/2) of a tile whose 16-byte chunk c of row r sits in
// physical chunk c ^ swz(r), for several swizzles and row pitches.
//
// Build and run (from the repository root; rocprofv3 from /tmp with TMPDIR=/tmp):
//   hipcc --offload-arch=gfx950 -O2 -std=c++17 flash-mlm_amd/probes/lds_swizzle_probe.hip -o <out>/lds_swizzle_probe
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS GRBM_GUI_ACTIVE --output-format csv \
//     -d <out>/pmc -o pmc -- <out>/lds_swizzle_probe > <out>/probe.log
//   python flash-mlm_amd/probes/lds_swizzle_report.py <out>/probe.log <out>/pmc/pmc_counter_collection.csv
// The program prints one line per dispatch ("pattern i name"), in launch order.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#define LDSP __attribute__((address_space(3)))
constexpr int ITER = 1024;

// fill the 64 KiB buffer, then read the lane's table address ITER x 4 times
__global__ __launch_bounds__(256) void probe_b128(const uint32_t* __restrict__ table, uint32_t* out) {
  __shared__ __align__(16) char lds[65536];
  for (int i = threadIdx.x; i < 65536 / 4; i += 256) ((uint32_t*)lds)[i] = i * 2654435761u;
  __syncthreads();
  const uint32_t a = table[threadIdx.x & 63] & 65535u & ~15u;
  const uint32_t base = (uint32_t)(uintptr_t)(LDSP char*)lds;
  uint32_t acc = 0;
  for (int it = 0; it < ITER; ++it) {
    u32x4 v0, v1, v2, v3;
    asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4\n\tds_read_b128 %2, %4\n\tds_read_b128 %3, %4\n\ts_waitcnt lgkmcnt(0)"
                 : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3) : "v"(base + a));
    acc ^= v0[0] ^ v1[1] ^ v2[2] ^ v3[3];
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}
__global__ __launch_bounds__(256) void probe_tr16(const uint32_t* __restrict__ table, uint32_t* out) {
  __shared__ __align__(16) char lds[65536];
  for (int i = threadIdx.x; i < 65536 / 4; i += 256) ((uint32_t*)lds)[i] = i * 2654435761u;
  __syncthreads();
  const uint32_t a = table[threadIdx.x & 63] & 65535u & ~7u;
  const uint32_t base = (uint32_t)(uintptr_t)(LDSP char*)lds;
  uint32_t acc = 0;
  for (int it = 0; it < ITER; ++it) {
    u32x2 v0, v1, v2, v3;
    asm volatile("ds_read_b64_tr_b16 %0, %4\n\tds_read_b64_tr_b16 %1, %4\n\tds_read_b64_tr_b16 %2, %4\n\tds_read_b64_tr_b16 %3, %4\n\ts_waitcnt lgkmcnt(0)"
                 : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3) : "v"(base + a));
    acc ^= v0[0] ^ v1[1] ^ v2[0] ^ v3[1];
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}

int main() {
  struct Swz {
    const char* name;
    std::function<int(int)> f;
  };
  const std::vector<Swz> swz = {
      {"kv_swz<D>=128> (r&3)<<1 ^ 9*b2 ^ 12*b3", [](int r) { return ((r & 3) << 1) ^ (((r >> 2) & 1) * 9) ^ (((r >> 3) & 1) * 12); }},
      {"former ((r&7)<<1)|((r>>3)&1)", [](int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }},
      {"k_swz<D>=128> r&15", [](int r) { return r & 15; }},
  };
  struct Pat {
    std::string name;
    std::function<uint32_t(int)> addr;
    bool tr16;
  };
  std::vector<Pat> pats;
  for (const Swz& s : swz)
    for (int rowb : {256, 512, 1024}) {
      auto f = s.f;
      for (int kc = 0; kc < 4; ++kc)
        pats.push_back({std::string("b128 K ") + s.name + " rowB=" + std::to_string(rowb) + " kc=" + std::to_string(kc),
                        [=](int l) { const int l16 = l & 15, g = l >> 4;
                                     return (uint32_t)(l16 * rowb + 16 * (((4 * kc + g) ^ f(l16)) & 15)); }, false});
      for (int db = 0; db < 4; ++db)
        pats.push_back({std::string("tr16 V ") + s.name + " rowB=" + std::to_string(rowb) + " db=" + std::to_string(db),
                        [=](int l) { const int l16 = l & 15, g = l >> 4, vr = 4 * g + (l16 >> 2), x = (l16 & 3) >> 1;
                                     return (uint32_t)(vr * rowb + 16 * (((2 * db + x) ^ f(vr)) & 15) + 8 * (l16 & 1)); }, true});
    }
  uint32_t *d = nullptr, *tab = nullptr;
  if (hipMalloc(&d, 2048 * 256 * 4) != hipSuccess || hipMalloc(&tab, 64 * 4) != hipSuccess) return 1;
  for (size_t p = 0; p < pats.size(); ++p) {
    uint32_t h[64];
    for (int l = 0; l < 64; ++l) h[l] = pats[p].addr(l);
    if (hipMemcpy(tab, h, sizeof h, hipMemcpyHostToDevice) != hipSuccess) return 1;
    if (pats[p].tr16)
      hipLaunchKernelGGL(probe_tr16, dim3(2048), dim3(256), 0, 0, tab, d);
    else
      hipLaunchKernelGGL(probe_b128, dim3(2048), dim3(256), 0, 0, tab, d);
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    printf("pattern %zu %s\n", p, pats[p].name.c_str());
  }
  return hipFree(d) == hipSuccess && hipFree(tab) == hipSuccess ? 0 : 1;
}
