// Issue cost of 16-byte-per-lane loads on one MI355X (gfx950): LDS-DMA
// (buffer_load_dwordx4 ... lds) against buffer_load_dwordx4 into VGPRs.
// Diagnostic only (not part of the library).  One workgroup of 4 wavefronts
// per CU; 1 or all 4 wavefronts of it issue a burst of 8 loads of 1 KB each
// and time the issue alone with s_memtime, then wait for the data; 2000
// bursts per wavefront from a 64 KB slice per workgroup (L2-resident after
// the first pass).  Offsets stay inside the slice and LDS writes inside the
// workgroup's 32 KB array.
//
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       jax-mlx-plugin_amd/probes/load_issue_rate.hip -o /tmp/load_issue_rate && /tmp/load_issue_rate
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kSlice = 65536;  // source bytes per workgroup
constexpr int kBursts = 2000;

template <bool LDS, int NWAVES>
__global__ __launch_bounds__(256) void issue_kernel(const unsigned* src, unsigned long long* cycles, unsigned* sink) {
  __shared__ __attribute__((aligned(16))) u32x4 lds[2048];  // 32 KB: 4 wavefronts x 8 loads x 1 KB
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  char* slice = const_cast<char*>(reinterpret_cast<const char*>(src)) + (size_t)blockIdx.x * kSlice;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(slice, (short)0, kSlice, 0x00020000);
  unsigned long long total = 0;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int r = 0; r < kBursts; ++r) {
    if (wave < NWAVES) {
      const unsigned long long c0 = __builtin_amdgcn_s_memtime();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      u32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // bytes (wave*8 + i) KB + 16*lane of one half of the slice
        const unsigned off = (unsigned)((wave * 8 + i) * 1024 + lane * 16 + (r & 1) * (kSlice / 2));
        if constexpr (LDS)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(lds + (wave * 8 + i) * 64), 16, off, 0, 0, 0);
        else
          v[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
      }
      const unsigned long long c1 = __builtin_amdgcn_s_memtime();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      total += c1 - c0;
      if constexpr (!LDS) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc ^= v[i];
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the burst has landed
    }
    __syncthreads();
  }
  if (lane == 0 && wave < NWAVES) cycles[blockIdx.x * 4 + wave] = total;
  sink[blockIdx.x * 256 + threadIdx.x] = LDS ? lds[threadIdx.x].x : (acc.x ^ acc.y ^ acc.z ^ acc.w);
}

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

template <bool LDS, int NW>
void run(const unsigned* src, unsigned long long* cycles, unsigned* sink, int blocks) {
  std::vector<unsigned long long> h(blocks * 4);
  for (int rep = 0; rep < 2; ++rep) {  // the first run warms L2 and the clocks
    hipLaunchKernelGGL((issue_kernel<LDS, NW>), dim3(blocks), dim3(256), 0, 0, src, cycles, sink);
    check(hipGetLastError(), "launch");
    check(hipDeviceSynchronize(), "sync");
  }
  check(hipMemcpy(h.data(), cycles, h.size() * 8, hipMemcpyDeviceToHost), "hipMemcpy");
  std::vector<unsigned long long> v;
  for (int b = 0; b < blocks; ++b)
    for (int w = 0; w < NW; ++w) v.push_back(h[b * 4 + w]);
  std::sort(v.begin(), v.end());
  const double burst = (double)v[v.size() / 2] / kBursts;  // median wavefront
  std::printf("| %-30s | %d | %6.1f | %5.1f |\n", LDS ? "buffer_load_dwordx4 ... lds" : "buffer_load_dwordx4 -> VGPRs", NW,
              burst, burst / 8);
}

}  // namespace

int main() {
  hipDeviceProp_t prop;
  check(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties");
  const int blocks = prop.multiProcessorCount;
  unsigned* src = nullptr;
  unsigned long long* cycles = nullptr;
  unsigned* sink = nullptr;
  check(hipMalloc(&src, (size_t)blocks * kSlice), "hipMalloc");
  check(hipMemset(src, 1, (size_t)blocks * kSlice), "hipMemset");
  check(hipMalloc(&cycles, (size_t)blocks * 4 * 8), "hipMalloc");
  check(hipMalloc(&sink, (size_t)blocks * 256 * 4), "hipMalloc");
  std::printf("%s, %d CUs, one workgroup per CU\n\n", prop.gcnArchName, blocks);
  std::printf("| load (8 per burst, 1 KB each) | wavefronts issuing per CU | cycles per burst | per instruction |\n");
  std::printf("|---|---:|---:|---:|\n");
  run<true, 1>(src, cycles, sink, blocks);
  run<false, 1>(src, cycles, sink, blocks);
  run<true, 4>(src, cycles, sink, blocks);
  run<false, 4>(src, cycles, sink, blocks);
  return 0;
}
