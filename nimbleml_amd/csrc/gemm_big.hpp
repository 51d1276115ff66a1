// Main loop of the fp16 MFMA GEMMs with operands staged by direct-to-LDS loads, shared by
// the prefill projections (ops_gemm.hip) and the float16 backward (ops_train.hip).
//
// A workgroup of 8 waves (2 per SIMD, so one multiplies while the other waits) owns a
// TM × TN output tile; wave w owns rows (w / 4)·TM/2 … and columns (w % 4)·TN/4 … as
// IA × JB MFMA 32×32×16 tiles. Both operands are k-contiguous rows (A: M rows, B: N
// rows). K advances in stages of 64 columns, double-buffered in LDS: a stage holds the
// TM + TN rows of the tile as whole 128-byte rows, written by global_load_lds_dwordx4
// (lane l of a wave writes bytes 16l…16l+15 of a 1 KiB block of 8 rows).
// The compiler cannot tell which buffer an LDS read touches, and it would wait for every
// outstanding direct-to-LDS load before each one (and before every workgroup barrier).
// So the waits are explicit: a raw s_barrier after s_waitcnt vmcnt(0) publishes a stage
// and frees the buffer of the stage before it, and fragment reads are ds_read_b128
// statements whose results pass through the s_waitcnt lgkmcnt that guards them. The
// next 16-wide k step's fragments are read while the current step's MFMAs run.
// The 16-byte chunk c of stage row r sits at position c ^ ((r / 2) & 7): the 16 lanes of
// a ds_read_b128 phase (rows r…r+15, one chunk) then cover all 64 banks once.
#pragma once

#include "kernels.hpp"

namespace nml {
namespace big {

constexpr int kK = 64;          // k columns per stage (128-byte rows)
constexpr int kStages = 2;
constexpr int kThreads = 512;   // 8 waves

template <int TM, int TN>
struct Shape {
  static_assert((TM == 256 || TM == 128) && (TN == 256 || TN == 128), "tile");
  static constexpr int IA = TM / 64;   // 32-row MFMA tiles per wave
  static constexpr int JB = TN / 128;  // 32-column MFMA tiles per wave
  static constexpr int StageBytes = (TM + TN) * kK * 2;
  static constexpr size_t Lds = static_cast<size_t>(kStages) * StageBytes;
};

__device__ __forceinline__ uint32_t swz_off(int row, int chunk) {
  return static_cast<uint32_t>(row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4));
}

__device__ __forceinline__ half8 lds_read16(uint32_t addr) {
  half8 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// Workgroup b runs on XCD b % 8; the workgroups of one XCD take one contiguous range of
// the `tiles` indices (any count: the first tiles % 8 XCDs take one more).
__device__ __forceinline__ int xcd_tile(int b, int tiles) {
  const int per = tiles >> 3, rem = tiles & 7, x = b & 7;
  return x * per + (x < rem ? x : rem) + (b >> 3);
}

// s_waitcnt lgkmcnt(IA + JB) (the step just issued may stay outstanding) or lgkmcnt(0),
// with the fragments passed through so that no use is moved above the wait.
template <int IA, int JB>
struct Lgkm;
template <>
struct Lgkm<4, 2> {
  static __device__ __forceinline__ void prev(half8 (&fa)[4], half8 (&fb)[2]) {
    asm volatile("s_waitcnt lgkmcnt(6)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1]));
  }
  static __device__ __forceinline__ void all(half8 (&fa)[4], half8 (&fb)[2]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1]));
  }
};
template <>
struct Lgkm<2, 1> {
  static __device__ __forceinline__ void prev(half8 (&fa)[2], half8 (&fb)[1]) {
    asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(fa[0]), "+v"(fa[1]), "+v"(fb[0]));
  }
  static __device__ __forceinline__ void all(half8 (&fa)[2], half8 (&fb)[1]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fa[0]), "+v"(fa[1]), "+v"(fb[0]));
  }
};

// acc[i][j] += Σ_k A[row a_i][k] · B[row b_j][k] over k in [k0, k0 + S·kK) (transposed
// when TR), for this wave's 32×32 tiles at rows m0 + (wave / 4)·TM/2 + 32i and columns
// n0 + (wave % 4)·TN/4 + 32j. Rows past M or N read row M-1 / N-1 (the caller stores
// none of them); the k range must lie inside both operands. S ≥ 1.
// TR: the accumulators hold the transposed tiles, D[n][m] (the operands of each MFMA
// swapped), so that in the D layout a lane holds one output row and runs of consecutive
// columns.
template <int TM, int TN, bool TR = false>
__device__ __forceinline__ void mainloop(const half_t* __restrict__ A, long long lda,
                                         const half_t* __restrict__ B, long long ldb, int M, int N,
                                         int k0, int S, int m0, int n0, char* lds_raw,
                                         floatx16 (&acc)[TM / 64][TN / 128]) {
  typedef Shape<TM, TN> Sh;
  constexpr int IA = Sh::IA, JB = Sh::JB, SB = Sh::StageBytes;
  constexpr int QA = TM / 64, QB = TN / 64;  // 8-row blocks per wave and stage
  constexpr int QM = QA > QB ? QA : QB;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_raw));

  // Lane l of block q carries row 8q + l/8 at chunk position l % 8, i.e. global chunk
  // (l % 8) ^ ((row / 2) & 7).
  const int lrow = lane >> 3, lpos = lane & 7;
  auto issue = [&](int s) {
    const int kc = k0 + s * kK;
    char* stage = lds_raw + (s % kStages) * SB;
#pragma unroll
    for (int j = 0; j < QM; ++j) {
      if (j < QA) {
        const int q = wave * QA + j;
        const int row = 8 * q + lrow;
        const int ch = lpos ^ ((row >> 1) & 7);
        const long long gr = m0 + row < M ? m0 + row : M - 1;
        // (address-space casts: global source, LDS destination)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(A + gr * lda + kc + ch * 8),
                                         (__attribute__((address_space(3))) void*)(stage + q * 1024), 16, 0, 0);
      }
      if (j < QB) {
        const int q = wave * QB + j;
        const int row = 8 * q + lrow;
        const int ch = lpos ^ ((row >> 1) & 7);
        const long long gr = n0 + row < N ? n0 + row : N - 1;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(B + gr * ldb + kc + ch * 8),
                                         (__attribute__((address_space(3))) void*)(stage + TM * 128 + q * 1024),
                                         16, 0, 0);
      }
    }
  };

  uint32_t offa[IA], offb[JB];
#pragma unroll
  for (int i = 0; i < IA; ++i) offa[i] = static_cast<uint32_t>(wm * (TM / 2) + i * 32 + (lane & 31));
#pragma unroll
  for (int j = 0; j < JB; ++j) offb[j] = static_cast<uint32_t>(wn * (TN / 4) + j * 32 + (lane & 31));

  // Stage t's barrier (every wave's loads of t landed, every wave done reading t - 1) is
  // followed by the loads of stage t + 1 into t - 1's buffer; before a stage's last step
  // each wave has its fragments in registers, so the next barrier may release the buffer.
  // With 256 × 256 tiles the waves sharing a SIMD (w and w + 4) issue at different times:
  // waves 0-3 after the barrier, waves 4-7 after their first k step's MFMAs (the stage's
  // loads issued in one burst by all eight waves stalled every SIMD's MFMAs at once:
  // C5 0.0490 → 0.0479 s and 0.0505 → 0.0497 s per compute_loss in A/Bs on two boxes;
  // staggering the 128 × 128 tiles too made the fp16 training step 1.6 % slower).
  constexpr bool kStagger = TM == 256 && TN == 256;
  auto wait_stage = [&](int t) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (t + 1 < S && (!kStagger || wave < 4)) issue(t + 1);
  };
  half8 fa0[IA], fb0[JB], fa1[IA], fb1[JB];
  auto read = [&](half8 (&fa)[IA], half8 (&fb)[JB], int t, int kk) {
    const uint32_t base = lds0 + static_cast<uint32_t>((t % kStages) * SB);
    const int ch = 2 * kk + (lane >> 5);
#pragma unroll
    for (int i = 0; i < IA; ++i) fa[i] = lds_read16(base + swz_off(offa[i], ch));
#pragma unroll
    for (int j = 0; j < JB; ++j) fb[j] = lds_read16(base + TM * 128 + swz_off(offb[j], ch));
  };
  auto mma = [&](const half8 (&fa)[IA], const half8 (&fb)[JB]) {
#pragma unroll
    for (int i = 0; i < IA; ++i)
#pragma unroll
      for (int j = 0; j < JB; ++j)
        acc[i][j] = TR ? __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[j], fa[i], acc[i][j], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
  };
  typedef Lgkm<IA, JB> W;
  issue(0);
  wait_stage(0);
  read(fa0, fb0, 0, 0);
  // Stages with a successor, then the last stage without the next stage's first read:
  // on every path (the loop's back edge and its exit alike) the reads issued at the bottom
  // meet the wait at the top of the next body before any use, and no path leaves the
  // main loop with reads still in flight (the caller's epilogue reuses their registers).
  auto body = [&](int s) {
    read(fa1, fb1, s, 1);
    W::prev(fa0, fb0);
    mma(fa0, fb0);
    if (kStagger && s + 1 < S && wave >= 4) issue(s + 1);  // stage s + 1 (see wait_stage)
    read(fa0, fb0, s, 2);
    W::prev(fa1, fb1);
    mma(fa1, fb1);
    read(fa1, fb1, s, 3);
    W::prev(fa0, fb0);
    mma(fa0, fb0);
    // Every MFMA of the third k step issues before the stage barrier below: left free, the
    // compiler moves half of them past it, where no wave of the workgroup can issue them
    // while the barrier waits (C5: 0.0529–0.0533 → 0.0507–0.0514 s per compute_loss in an
    // A/B on one box).
#pragma unroll
    for (int i = 0; i < IA; ++i)
#pragma unroll
      for (int j = 0; j < JB; ++j) asm volatile("" : "+v"(acc[i][j]));
    W::all(fa1, fb1);
  };
  int s = 0;
  for (; s + 1 < S; ++s) {
    body(s);
    wait_stage(s + 1);
    read(fa0, fb0, s + 1, 0);
    mma(fa1, fb1);
  }
  body(s);
  mma(fa1, fb1);
}

}  // namespace big
}  // namespace nml
