// f32 GEMM tile kernel on v_mfma_f32_32x32x2_f32, shared by the static
// kernels of gemm_f32.hip (plain store) and the hipRTC kernels of
// gemm_jit.cpp (a fused elementwise program applied to the accumulators).
// Self-contained: under hipRTC it is compiled from its text, with no other
// header.
//
//   C[b][m][n] = sum_k A[b][m][k] * B[b][k][n]     (row-major, fp32)
//
// Tiling (MI355X, 256 CUs, 64-wide wavefronts, 160 KB LDS per CU):
// - a workgroup computes a BM x BN tile with (BM/32) x (BN/64) wavefronts,
//   each a 32 x 64 block as two 32x32 MFMA accumulators (32 VGPRs);
// - K advances in 32-wide k-tiles staged through S LDS stages by buffer
//   loads to LDS (16 bytes per lane, no VGPR staging).  A k-tile row of A is
//   128 bytes (8 chunks of 16); chunk c of row r sits at slot c ^ swz(r), so
//   the MFMA operand reads (16 lanes on 16 rows, one chunk each) hit every
//   bank once whether the LDS serves 128 or 256 bytes per clock.  A k-tile
//   row of B is BN floats, stored as loaded;
// - k order inside an 8-wide group is permuted: lane half h of the MFMA at
//   step s holds k = 8q + 4h + s, so one ds_read_b128 gives an A lane its
//   four k values of the group, and B is read as float2 pairs (two adjacent
//   columns, one per accumulator) from the row k.  The sum is over the same
//   products; only the fp32 accumulation order differs from a sequential
//   loop;
// - fragments of group q+1 are read while the MFMAs of group q run, and the
//   k-tile switch (wait for this wave's loads, barrier, next loads, first
//   reads of the next tile) sits halfway through the last group's MFMAs.
// Out-of-range reads come back as zeros (buffer range checks): rows past M,
// k-rows of B past K; A chunks past K are pointed out of range explicitly.
// The hardware checks only the per-lane (VGPR) offset of a raw buffer load
// against the resource's extent, not the scalar offset, so every row step
// lives in the per-lane offset and the k-tile position moves the resource
// base (its extent shrinking by the same amount): no load can reach past
// A's first min(M - m0, BM) rows of the tile or past B's last element,
// B[K-1][N-1].  Columns past N are computed from whatever the loads return
// (elements of B's next row, or zeros on its last row) and never stored.
//
// Requirements checked by the host: K % 4 == 0, N % 4 == 0, lda and ldb
// multiples of 4, A and B 16-byte aligned, C 8-byte aligned, and the byte
// offsets a k-tile load forms (BM * lda * 4, K * ldb * 4) below 2^31.
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

namespace mfx_gemm_tile {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;

struct Params {
  const float* a;
  const float* b;
  float* c;
  long long sa, sb, sc;  // batch strides (elements)
  int M, N, K;
  int lda, ldb, ldc;
  int tiles_m, tiles_n;
};

constexpr int kBK = 32;  // k-tile
constexpr int kWM = 32;  // wavefront block rows
constexpr int kWN = 64;  // wavefront block columns (two 32-wide accumulators)

__host__ __device__ constexpr int threads(int BM, int BN) { return (BM / kWM) * (BN / kWN) * 64; }
__host__ __device__ constexpr int lds_bytes(int BM, int BN, int S) { return S * (BM + BN) * kBK * 4; }

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

template <int N>
struct Int {
  static constexpr int value = N;
};
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(Int<B>{});
    static_for<B + 1, E>(f);
  }
}

// s_waitcnt with only vmcnt = n (n < 64); expcnt and lgkmcnt untouched.
template <int n>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 0xF) | ((n >> 4) << 14));
}
// vmcnt = n and lgkmcnt = 0.
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  __builtin_amdgcn_s_waitcnt(0x0070 | (n & 0xF) | ((n >> 4) << 14));
}

// The epilogue type E provides
//   struct Args;                       (kernel argument block)
//   struct Col;                        (per-lane state of the lane's column pair)
//   struct Row;                        (values loaded for one row of the pair)
//   static Col col(const Params&, const Args&, int n);
//   static Row row(const Params&, const Args&, const Col&, int b, int m, int n);
//   static void store(const Params&, const Args&, const Col&, const Row&, int b, int m, int n,
//                     float v0, float v1);
// col() runs before the k loop (its loads complete under the MFMAs); row()
// runs for the lane's 16 rows back to back after it, all loads in flight at
// once; store() receives C[b][m][n] and C[b][m][n+1] and runs for m < M and
// n < N only.  col() and row() are called with indices clamped into the
// matrix (n <= N - 2, m <= M - 1), so they need no bounds checks.
template <int BM, int BN, int S, class E>
__device__ __forceinline__ void gemm_tile(const Params& p, const typename E::Args& ea) {
  constexpr int NW = (BM / kWM) * (BN / kWN);
  constexpr int QN = kBK / 8;
  constexpr int A_BYTES = BM * kBK * 4, B_BYTES = kBK * BN * 4;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_LOADS = A_BYTES / 1024 / NW;
  constexpr int B_LOADS = B_BYTES / 1024 / NW;
  constexpr int LOADS = A_LOADS + B_LOADS;
  constexpr int A_ROWS = 1024 / (kBK * 4);  // A rows per load instruction
  constexpr int B_ROWS = 1024 / (BN * 4);   // B k-rows per load instruction
  static_assert(A_LOADS * NW * 1024 == A_BYTES && B_LOADS * NW * 1024 == B_BYTES, "loads cover the tile");
  static_assert(B_ROWS >= 1 && BN % kWN == 0 && BM % kWM == 0, "tile shape");
  static_assert(S >= 2, "at least two stages");
  __shared__ __attribute__((aligned(1024))) char smem[S * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroups go to the 8 XCDs round-robin; give each XCD a contiguous run
  // of tiles (row-major over tiles), so the tiles sharing an A row block or
  // a B column block meet in the same L2.
  const int ntiles = p.tiles_m * p.tiles_n;
  const int w = blockIdx.x;
  const int tile = ntiles % 8 == 0 ? (w % 8) * (ntiles / 8) + w / 8 : w;
  const int tm = tile / p.tiles_n, tn = tile % p.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int bz = blockIdx.y;
  const float* A = p.a + (long long)bz * p.sa;
  const float* B = p.b + (long long)bz * p.sb;

  // A loader: instruction i of wave w fills rows (i*NW + w)*A_ROWS + lane/8,
  // chunk slot lane%8 from source chunk slot ^ swz(row).  The resource of
  // k-tile t starts at A[m0][t*kBK] and spans the tile's rows below M
  // (a_span bytes from A[m0][0]) minus that start.
  const int a_rows = p.M - m0 < BM ? p.M - m0 : BM;
  const int a_span = a_rows * p.lda * 4;
  const char* a_base = (const char*)(A + (long long)m0 * p.lda);
  const int a_row = wave * A_ROWS + lane / 8;
  const int a_chunk = (lane & 7) ^ swz(a_row);
  unsigned a_vo[A_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i)
    a_vo[i] = (unsigned)(((i * NW * A_ROWS + a_row) * p.lda + a_chunk * 4) * 4);
  // B loader: instruction i of wave w fills k-rows (i*NW + w)*B_ROWS + lane/(BN/4);
  // the resource of k-tile t starts at B[t*kBK][0] and ends at B's last
  // element (N % 4 == 0, so no 16-byte load straddles that end).
  const int b_span = ((p.K - 1) * p.ldb + p.N) * 4;
  const int b_row = wave * B_ROWS + lane / (BN / 4);
  unsigned b_vo[B_LOADS];
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i)
    b_vo[i] = (unsigned)((((i * NW * B_ROWS + b_row) * p.ldb) + n0 + (lane % (BN / 4)) * 4) * 4);
  const int T = (p.K + kBK - 1) / kBK;

  auto issue = [&](int t, int stage) {
    char* sa = smem + stage * STAGE;
    char* sb = sa + A_BYTES;
    const bool a_in = t * kBK + a_chunk * 4 < p.K;
    const int a_off_t = t * kBK * 4, b_off_t = t * kBK * p.ldb * 4;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a_base + a_off_t), (short)0, a_span - a_off_t, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)((const char*)B + b_off_t), (short)0, b_span - b_off_t, 0x00020000);
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sa + (i * NW + wave) * 1024), 16,
                                               a_in ? a_vo[i] : 0x80000000u, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(sb + (i * NW + wave) * 1024), 16, b_vo[i], 0,
                                               0, 0);
  };

  const int wm0 = (wave / (BN / kWN)) * kWM, wn0 = (wave % (BN / kWN)) * kWN;
  const int li = lane & 31, h = lane >> 5;
  unsigned a_off[QN];
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int row = wm0 + li;
    a_off[q] = (unsigned)(row * (kBK * 4) + (((2 * q + h) ^ swz(row)) * 16));
  }
  const unsigned b_off = (unsigned)(A_BYTES + (4 * h) * (BN * 4) + (wn0 + 2 * li) * 4);

  // Columns of this lane: wn0 + 2li (acc0) and wn0 + 2li + 1 (acc1).
  const int n = n0 + wn0 + 2 * li;
  const int n_ld = n < p.N ? n : p.N - 2;
  const typename E::Col cs = E::col(p, ea, n_ld);

  f32x16 acc0 = {}, acc1 = {};
  f32x4 fa[2];
  f32x2 fb[2][4];
  auto read = [&](int stage, int q, int buf) {
    const char* base = smem + stage * STAGE;
    fa[buf] = *(const f32x4*)(base + a_off[q]);
#pragma unroll
    for (int s = 0; s < 4; ++s) fb[buf][s] = *(const f32x2*)(base + b_off + (8 * q + s) * (BN * 4));
  };
  // MFMA j of a group: k step j/2, accumulator j%2.
  auto mfma = [&](int buf, int j) {
    const int s = j >> 1;
    if (j & 1) acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[buf][s], fb[buf][s][1], acc1, 0, 0, 0);
    else acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[buf][s], fb[buf][s][0], acc0, 0, 0, 0);
  };
  constexpr int MG = 8;  // MFMAs per group

#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < T) issue(s, s);
  // k-tile 0 has landed (this wave's loads, then everyone's); the later
  // stages stay in flight.
  if (T >= S) wait_vm<LOADS * (S - 1)>();
  else wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  fence();
  read(0, 0, 0);

  for (int t = 0; t < T; ++t) {
    const int stage = t % S;
    static_for<0, QN>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      constexpr int buf = q % 2;
      if constexpr (q < QN - 1) {
        fence();
        read(stage, q + 1, buf ^ 1);
        fence();
#pragma unroll
        for (int j = 0; j < MG; ++j) mfma(buf, j);
      } else {
#pragma unroll
        for (int j = 0; j < MG / 2; ++j) mfma(buf, j);
        fence();
        // This group's reads landed long ago; waiting for them here keeps
        // the compiler from waiting for the next tile's reads below.
        __builtin_amdgcn_s_waitcnt(0xC07F);
        fence();
        if (t + 1 < T) {
          // Tile t+1 has landed (this wave's loads, then everyone's), and
          // every wave is done reading tile t, whose stage the loads of
          // tile t+S reuse.
          if (S > 2 && T - 2 - t >= S - 2) wait_vm_lgkm0<LOADS * (S > 2 ? S - 2 : 0)>();
          else wait_vm_lgkm0<0>();
          __builtin_amdgcn_s_barrier();
          fence();
          if (t + S < T) issue(t + S, stage);
          read((t + 1) % S, 0, buf ^ 1);
          fence();
        }
#pragma unroll
        for (int j = MG / 2; j < MG; ++j) mfma(buf, j);
      }
    });
  }

  // Accumulator element e of lane (li, h): row 8*(e/4) + 4h + e%4 of the
  // wavefront block.
  typename E::Row rows[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int m = m0 + wm0 + 8 * (e / 4) + 4 * h + (e & 3);
    rows[e] = E::row(p, ea, cs, bz, m < p.M ? m : p.M - 1, n_ld);
  }
  if (n < p.N) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + wm0 + 8 * (e / 4) + 4 * h + (e & 3);
      if (m < p.M) E::store(p, ea, cs, rows[e], bz, m, n, acc0[e], acc1[e]);
    }
  }
}

// Plain store: C[b][m][n..n+1] at c + b*sc + m*ldc + n.
struct StoreEpilogue {
  struct Args {};
  struct Col {};
  struct Row {};
  static __device__ __forceinline__ Col col(const Params&, const Args&, int) { return Col{}; }
  static __device__ __forceinline__ Row row(const Params&, const Args&, const Col&, int, int, int) { return Row{}; }
  static __device__ __forceinline__ void store(const Params& p, const Args&, const Col&, const Row&, int b, int m,
                                               int n, float v0, float v1) {
    f32x2 v = {v0, v1};
    *(f32x2*)(p.c + (long long)b * p.sc + (long long)m * p.ldc + n) = v;
  }
};

}  // namespace mfx_gemm_tile
