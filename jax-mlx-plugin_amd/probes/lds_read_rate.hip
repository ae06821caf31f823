// LDS read rate on one MI355X (gfx950), per instruction form: how many CU
// cycles one wavefront-wide LDS read takes when every SIMD keeps reads in
// flight.  Diagnostic only (not part of the library); the attention kernels'
// cost model rests on it:
//   - ds_read_b32 / ds_read_b64 / ds_read_b128, lanes on consecutive
//     addresses;
//   - ds_read_b64_tr_b16 with the flash kernels' V^T operand addresses
//     (64-key x 128-feature bf16 tile, XOR-swizzled 16-byte chunks).
// Each wavefront issues 16 reads, waits once for all of them, folds them
// into a checksum and repeats; it times its loop with s_memtime (shader
// clock).  8 or 16 wavefronts per CU (2 or 4 workgroups of 4).
//
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       jax-mlx-plugin_amd/probes/lds_read_rate.hip -o /tmp/lds_read_rate && /tmp/lds_read_rate
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kLdsBytes = 32 * 1024;  // per workgroup: four fit on a CU
constexpr int kReads = 16;            // reads in flight per wavefront
constexpr int kIters = 1024;

enum Form { kB32 = 0, kB64 = 1, kB128 = 2, kTrV = 3 };

// Byte offset of read j of lane `lane` in iteration `rot` (rotation keeps
// the addresses moving); always inside [0, kLdsBytes) and aligned to the
// form's width.
template <int FORM>
__device__ unsigned offset(unsigned lane, int j, unsigned rot) {
  constexpr unsigned mask = kLdsBytes - 1;
  if constexpr (FORM == kB32) return (lane * 4 + j * 256 + rot) & (mask & ~3u);
  if constexpr (FORM == kB64) return (lane * 8 + j * 512 + rot) & (mask & ~7u);
  if constexpr (FORM == kB128) return (lane * 16 + j * 1024 + rot) & (mask & ~15u);
  // Transposing V^T read of the flash kernels: 16 lanes cover 4 tile rows x
  // 2 chunks; rows of 128 bf16 features, chunk slot c ^ swz(row).
  const int half = lane >> 5, tj = lane & 15, tg = (lane >> 4) & 1;
  const int row = 4 * half + (tj >> 2) + ((j & 8) ? 8 : 0);
  const int swz = (row & 3) | (((row ^ (row >> 2)) & 3) << 2);
  const int chunk = tg * 2 + ((tj & 3) >> 1), sub = (tj & 1) * 4;
  const int dt = j & 3, ks = (j >> 2) & 1;
  const unsigned in_tile = (unsigned)(((ks * 16 + row) * 128 + sub + ((dt * 4 + chunk) ^ swz) * 8) * 2);
  return (in_tile + rot) & (mask & ~7u);
}

template <int FORM>
__global__ __launch_bounds__(256) void lds_read_kernel(unsigned long long* cycles, unsigned* sink) {
  __shared__ __attribute__((aligned(16))) u32x4 lds[kLdsBytes / 16];
  const unsigned t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (unsigned i = t; i < kLdsBytes / 16; i += 256) lds[i] = u32x4{i, i + 1, i + 2, i + 3};
  __syncthreads();
  const unsigned base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  unsigned acc = 0;
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < kIters; ++it) {
    const unsigned rot = ((unsigned)it + wave) * 2048u;
    u32x4 r[kReads];
#pragma unroll
    for (int j = 0; j < kReads; ++j) {
      const unsigned a = base + offset<FORM>(lane, j, rot);
      if constexpr (FORM == kB32) {
        unsigned v;
        asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(a));
        r[j] = u32x4{v, 0u, 0u, 0u};
      } else if constexpr (FORM == kB64) {
        u32x2 v;
        asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(a));
        r[j] = u32x4{v.x, v.y, 0u, 0u};
      } else if constexpr (FORM == kB128) {
        asm volatile("ds_read_b128 %0, %1" : "=v"(r[j]) : "v"(a));
      } else {
        u32x2 v;
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(a));
        r[j] = u32x4{v.x, v.y, 0u, 0u};
      }
    }
    // One wait for all 16; the results are tied to it so nothing reads them
    // earlier.
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]),
                   "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11]), "+v"(r[12]), "+v"(r[13]), "+v"(r[14]),
                   "+v"(r[15]));
#pragma unroll
    for (int j = 0; j < kReads; ++j) acc ^= r[j].x ^ r[j].y ^ r[j].z ^ r[j].w;
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  if (lane == 0) cycles[blockIdx.x * 4 + wave] = c1 - c0;
  sink[blockIdx.x * 256 + t] = acc;
}

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

template <int FORM>
void run(int cus, int wgs_per_cu, const char* name, int bytes_per_lane) {
  const int blocks = wgs_per_cu * cus;
  unsigned long long* cycles = nullptr;
  unsigned* sink = nullptr;
  check(hipMalloc(&cycles, (size_t)blocks * 4 * sizeof(unsigned long long)), "hipMalloc");
  check(hipMalloc(&sink, (size_t)blocks * 256 * sizeof(unsigned)), "hipMalloc");
  std::vector<unsigned long long> h(blocks * 4);
  for (int rep = 0; rep < 2; ++rep) {  // the first run warms the clocks
    hipLaunchKernelGGL(lds_read_kernel<FORM>, dim3(blocks), dim3(256), 0, 0, cycles, sink);
    check(hipGetLastError(), "launch");
    check(hipDeviceSynchronize(), "sync");
  }
  check(hipMemcpy(h.data(), cycles, h.size() * sizeof(h[0]), hipMemcpyDeviceToHost), "hipMemcpy");
  std::sort(h.begin(), h.end());
  const double cyc = (double)h[h.size() / 2];  // median wavefront
  const double instr_per_cu = (double)kReads * kIters * wgs_per_cu * 4;
  const double bytes_per_instr = 64.0 * bytes_per_lane;
  std::printf("| %-30s | %2d | %5.2f | %6.1f |\n", name, wgs_per_cu * 4, cyc / instr_per_cu,
              bytes_per_instr * instr_per_cu / cyc);
  check(hipFree(cycles), "hipFree");
  check(hipFree(sink), "hipFree");
}

}  // namespace

int main() {
  hipDeviceProp_t prop;
  check(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties");
  const int cus = prop.multiProcessorCount;
  std::printf("%s, %d CUs\n\n", prop.gcnArchName, cus);
  std::printf("| read (16 in flight per wavefront) | waves/CU | CU cycles per wave-wide read | B/clk/CU |\n");
  std::printf("|---|---:|---:|---:|\n");
  for (int wgs : {2, 4}) {
    run<kB32>(cus, wgs, "ds_read_b32, consecutive", 4);
    run<kB64>(cus, wgs, "ds_read_b64, consecutive", 8);
    run<kB128>(cus, wgs, "ds_read_b128, consecutive", 16);
    run<kTrV>(cus, wgs, "ds_read_b64_tr_b16, flash V^T", 8);
  }
  return 0;
}
