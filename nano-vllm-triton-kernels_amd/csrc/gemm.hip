// GEMM C = A @ B with fp32 accumulation for gfx950.
//
// Replaces nanovllm/kernels/matmul.py (Triton, :11-99): A [M, K], B [K, N] with arbitrary element strides
// (B = W.t() of an nn.Linear weight [N, K] is the common case), fp32 or bf16 inputs, C [M, N] in the input dtype.
// fp32 inputs: precision "ieee" uses them as they are, "tf32" rounds each input to a 10-bit mantissa
// (round to nearest even) before the products, which is what a tf32 tensor-core product sees.
//
// Kernels:
//   gemm_mfma_nt   bf16, A K-contiguous and B K-contiguous (sbk == 1; B = W.t() of a [N, K] weight) or, BNM,
//                  N-contiguous (sbn == 1; a row-major [K, N] B): 32x32x16 bf16 MFMA, register + LDS staged
//                  pipeline, GROUP_M-swizzled, XCD-aware tile order.
//   gemm_skinny    bf16 with M <= 32, same layout: 16 columns per block, K split over 8 waves, 16x16x32 MFMA.
//   gemm_mfma_f32  fp32, A K-contiguous, B K- or N-contiguous: 32x32x2 fp32 MFMA (exact products, fp32 sums).
//   gemm_generic   any dtype/strides/precision: 64x64 tile, 4x4 outputs per thread, fp32 FMA.
#include <type_traits>

#include "common.h"

namespace nvhip {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float round_tf32(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) return x;  // inf / nan unchanged
  u += 0xfffu + ((u >> 13) & 1u);
  return __uint_as_float(u & 0xffffe000u);
}

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }

struct GemmArgs {
  void* c;
  const void* a;
  const void* b;
  int64_t M, N, K;
  int64_t sam, sak, sbk, sbn, scm, scn;
};

// 64x64 output tile per 256-thread block; thread (ty, tx) owns rows ty + 16*i, cols tx + 16*j (i, j < 4).
// K is staged 16 at a time through LDS; out-of-range elements load as 0.
template <typename T, bool TF32>
__global__ __launch_bounds__(kBlock) void gemm_generic(const GemmArgs g) {
  constexpr int BM = 64, BN = 64, BK = 16;
  __shared__ float As[BK][BM + 1];
  __shared__ float Bs[BK][BN + 1];
  const T* A = static_cast<const T*>(g.a);
  const T* B = static_cast<const T*>(g.b);
  T* C = static_cast<T*>(g.c);
  const int64_t m0 = int64_t(blockIdx.y) * BM, n0 = int64_t(blockIdx.x) * BN;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < g.K; k0 += BK) {
    for (int i = threadIdx.x; i < BM * BK; i += kBlock) {
      const int r = i / BK, kk = i % BK;
      const int64_t m = m0 + r, k = k0 + kk;
      float v = (m < g.M && k < g.K) ? to_f32<T>(A[m * g.sam + k * g.sak]) : 0.0f;
      if constexpr (TF32) v = round_tf32(v);
      As[kk][r] = v;
    }
    for (int i = threadIdx.x; i < BN * BK; i += kBlock) {
      const int cidx = i % BN, kk = i / BN;
      const int64_t n = n0 + cidx, k = k0 + kk;
      float v = (n < g.N && k < g.K) ? to_f32<T>(B[k * g.sbk + n * g.sbn]) : 0.0f;
      if constexpr (TF32) v = round_tf32(v);
      Bs[kk][cidx] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
      if (m < g.M && n < g.N) C[m * g.scm + n * g.scn] = from_f32<T>(acc[i][j]);
    }
}


// ------------------------------------------------------------------------------------------------------------
// bf16 MFMA kernel (A and B K-contiguous with 16-byte aligned rows, C with unit column stride).
//
// Block tile BM x BN x 64 with WAVES_M x WAVES_N waves, each owning WM x WN outputs as FM x FN tiles of
// v_mfma_f32_32x32x16_bf16, issued with the operands swapped (its "A" is the B^T = W fragment, its "B" the A
// fragment), so that lane l's 16 accumulators of tile (fm, fn) hold output row m = fm*32 + l%32, columns
// n = fn*32 + 8*(r/4) + 4*(l/32) + r%4. Operand fragments (verified on gfx950): lane l reads row l%32,
// k = 8*(l/32) .. +8 of the 16-wide k step.
//
// Data path per k-tile of 64:
//   global -> VGPRs   16-byte loads, RS tiles in flight in registers (RS = 2 keeps 48-96 KB per block in flight,
//                     enough to cover the ~2000-cycle L2 latency measured at full load; 64x64 tiles, which run
//                     when there are few of them, use RS = 4)
//   VGPRs -> LDS      two LDS stages, [rows][64] bf16 per operand; 16-byte chunk c of row r stored at chunk
//                     c ^ ((r >> 1) & 7): with gfx950's 64 four-byte banks the 16 rows a half-wave fragment read
//                     touches land in 16 distinct 16-byte bank groups (conflict-free)
//   LDS -> MFMA       fragments for the next 16-wide k step are read while the current step's MFMAs issue
// The next k-tile's LDS writes and global loads are interleaved between the MFMAs (sched_group_barrier), and the
// one barrier per k-tile sits before its last k step (see `step`). The loop body is branch-free (a prefetch past
// the last tile re-reads it) so the compiler's wait counts keep the younger register stage in flight.
// Epilogue: accumulators -> bf16 -> LDS tile (row pitch BN + 8) -> 16-byte row-contiguous stores written through
// the L2 (store16_wt: the end-of-kernel L2 write-back then has no output lines to flush; M = 2048 qkv 22.9 -> 21.8
// us). Per-block timestamps of that launch: prologue (first k-tile) 1.5 us, main loop 12.5 us at a 1.9-2.0 GHz
// shader clock (2.35 GHz without the global loads), epilogue 2.3 us.
// Tile order: the block id is remapped so consecutive ids share an XCD (blocks are dealt round-robin over the 8
// XCDs), then mapped through the GROUP_M swizzle of the reference (matmul.py:50-57).
// Rows past M / columns past N are loaded clamped to the last row and never stored. With KTAIL, chunks past K
// load as zero (K a multiple of 8); otherwise K is a multiple of 64 * RS.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGroupM = 8;
constexpr int kBK = 64;

struct MfmaArgs {
  uint16_t* c;
  const uint16_t* a;
  const uint16_t* w;  // B^T: element (n, k) at w + n*swn + k; BNM kernels: B, element (k, n) at w + k*swn + n
  int M, N, K;
  int64_t sam, swn, scm;
  int splits = 1;      // PARTIAL kernels: K ranges; block b computes range b % splits of tile b / splits
  float* ws = nullptr; // PARTIAL kernels: fp32 partial products [splits, M, N]
};

__device__ __forceinline__ void tile_coords(int pid, int M, int N, int BM, int BN, int& pid_m, int& pid_n) {
  const int num_m = (M + BM - 1) / BM, num_n = (N + BN - 1) / BN;
  const int total = num_m * num_n;
  if (total % 8 == 0) {
    const int per_xcd = total / 8;
    pid = (pid % 8) * per_xcd + pid / 8;
  }
  const int in_group = kGroupM * num_n;
  const int first_m = (pid / in_group) * kGroupM;
  const int group_rows = min(num_m - first_m, kGroupM);
  pid_m = first_m + (pid % in_group) % group_rows;
  pid_n = (pid % in_group) / group_rows;
}

// step(kt + S, slot S) for S = 0 .. RS - 1: the k-tiles of one pass over the RS register slots.
template <int S, int RS, typename F>
__device__ __forceinline__ void unroll_steps(F& step, int kt) {
  if constexpr (S < RS) {
    step(kt + S, std::integral_constant<int, S>{});
    unroll_steps<S + 1, RS>(step, kt);
  }
}

// SILU: W is [2 * N2, K] = [gate; up] (N = 2 * N2) and C is [M, N2] = bf16(silu(A Wg^T)) * bf16(A Wu^T) rounded
// to bf16: a tile's first BN / 2 B rows are gate rows n0 / 2 .., the last BN / 2 the matching up rows N2 + n0 / 2 ..
// (so the per-column k order is that of the plain product, and the result is bitwise the unfused one).
// PARTIAL (split-K, for launches with few tiles): the block's K range is z * K / splits .. (z + 1) * K / splits and
// its fp32 tile goes unrounded to ws[z] (N a multiple of BN, K / splits a multiple of 64 * RS); the consumer sums
// the splits in order.
// BNM: B is N-contiguous ([K, N] rows of stride swn, N a multiple of 8; the layout of a plain row-major B). Its
// k-tile is staged as it lies, [64 k][BN n] with a row pitch of BN + 32 elements (rows 4 apart land 64 bytes apart
// in the 256-byte bank space), and the B^T fragment of a 16-wide k step (lane l: column l % 32, k = 8 (l / 32) ..
// +8) comes from two transpose reads ds_read_b64_tr_b16: lanes 4j + q of a 16-lane group address row kb + j,
// columns nb + 4q .. +4, and lane i receives column nb + i of rows kb .. kb + 3 (then kb + 4 .. kb + 7). The k order
// of every output, and so the result, is that of the K-contiguous kernel.
template <int BM, int BN, int WAVES_M, int WAVES_N, int RS, bool KTAIL, bool SILU = false, bool PARTIAL = false,
          bool BNM = false>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void gemm_mfma_nt(const MfmaArgs g) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N, FM = WM / 32, FN = WN / 32;
  static_assert(FM >= 1 && FN >= 1 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
  constexpr int AC = BM * 8 / NT, BC = BN * 8 / NT, CH = AC + BC;  // 16-byte chunks per thread per k-tile
  static_assert(AC >= 1 && BC >= 1 && AC * NT == BM * 8 && BC * NT == BN * 8, "tile too small for the block");
  static_assert(RS >= 1 && RS <= 8, "register stages");
  static_assert(!(BNM && (SILU || PARTIAL)), "N-contiguous B: plain products only");
  constexpr int BPITCH = BN + 32;                                      // BNM: row pitch of the staged B k-tile
  constexpr int STAGE = BM * kBK + (BNM ? kBK * BPITCH : BN * kBK);  // bf16 elements per LDS stage
  constexpr int OUT_PITCH = BN + 8;
  constexpr int LDS_ELEMS = (2 * STAGE > BM * OUT_PITCH) ? 2 * STAGE : BM * OUT_PITCH;
  constexpr int NMF = FM * FN;            // MFMAs per 16-wide k step
  constexpr int WPK = (CH + 2) / 3;       // next-tile chunks written to LDS per k step (k steps 0..2)
  constexpr int LPK = (CH + 3) / 4;       // chunks refilled from global memory per k step (k steps 0..3)
  __shared__ __attribute__((aligned(16))) uint16_t smem[LDS_ELEMS];

  int pid = blockIdx.x, z = 0;
  if constexpr (PARTIAL) {
    z = pid % g.splits;
    pid /= g.splits;
  }
  const int kspan = PARTIAL ? g.K / g.splits : g.K, kbeg = z * kspan;
  int pid_m, pid_n;
  tile_coords(pid, g.M, g.N, BM, BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // chunk i < AC: A chunk c = tid + NT*i; else B chunk c = tid + NT*(i-AC). Row c/8, logical k-chunk c%8, stored
  // in LDS at chunk (c%8) ^ ((row >> 1) & 7) of the row. BNM: B chunk c is k row c / (BN/8) of the k-tile, columns
  // 8 (c % (BN/8)) .. +8 (clamped into [0, N)), stored at the same place of the staged tile.
  const uint16_t* src[CH];
  int dst[CH], kofs[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const bool isA = i < AC;
    const int c = tid + NT * (isA ? i : i - AC), row = c / 8, kc = c % 8;
    if (BNM && !isA) {
      constexpr int CPRB = BN / 8;
      const int kr = c / CPRB, col = min(n0 + (c % CPRB) * 8, g.N - 8);
      src[i] = g.w + int64_t(kbeg + kr) * g.swn + col;
      dst[i] = BM * kBK + kr * BPITCH + (c % CPRB) * 8;
      kofs[i] = kr;
      continue;
    }
    int wrow = min(n0 + row, g.N - 1);
    if constexpr (SILU) {
      const int n2 = g.N / 2, half = BN / 2;
      wrow = row < half ? min(n0 / 2 + row, n2 - 1) : n2 + min(n0 / 2 + row - half, n2 - 1);
    }
    src[i] = (isA ? g.a + int64_t(min(m0 + row, g.M - 1)) * g.sam : g.w + int64_t(wrow) * g.swn) + kbeg + kc * 8;
    dst[i] = (isA ? 0 : BM * kBK) + row * kBK + ((kc ^ ((row >> 1) & 7)) * 8);
    kofs[i] = kc * 8;
  }
  auto gload1 = [&](int i, int k0) -> u32x4 {
    const int64_t step = (BNM && i >= AC) ? int64_t(k0) * g.swn : int64_t(k0);  // k0 rows of B, or k0 elements
    if (!KTAIL || k0 + kofs[i] < g.K) return *reinterpret_cast<const u32x4*>(src[i] + step);
    return u32x4{0, 0, 0, 0};
  };
  u32x4 r[RS][CH];
  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16_t{};

  const int frag_row = lane % 32, frag_half = lane / 32, swz = (frag_row >> 1) & 7;
  const int nk = (kspan + kBK - 1) / kBK;
  // prologue: k-tile 0 -> LDS stage 0; k-tiles 1..RS in flight in the register slots
#pragma unroll
  for (int i = 0; i < CH; ++i) r[0][i] = gload1(i, 0);
#pragma unroll
  for (int i = 0; i < CH; ++i) *reinterpret_cast<u32x4*>(smem + dst[i]) = r[0][i];
#pragma unroll
  for (int s = 0; s < RS; ++s)
#pragma unroll
    for (int i = 0; i < CH; ++i) r[s][i] = gload1(i, min(1 + s, nk - 1) * kBK);
  __syncthreads();

  bf16x8_t af[2][FM], bfr[2][FN];
  // BNM transpose reads: lane 4j + q of 16-lane group G addresses row 8 (G / 2) + j of the k step (and + 4),
  // columns 16 (G % 2) + 4 q of the fragment
  const int tr_row = 8 * (lane / 32) + (lane % 16) / 4, tr_col = 16 * ((lane / 16) & 1) + 4 * (lane % 4);
  auto load_frags = [&](const uint16_t* st, int kk, int fs) {
    const int chunk = ((2 * kk + frag_half) ^ swz) * 8;
#pragma unroll
    for (int i = 0; i < FM; ++i)
      af[fs][i] = *reinterpret_cast<const bf16x8_t*>(&st[(wm * WM + i * 32 + frag_row) * kBK + chunk]);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (BNM) {
        const uint16_t* p = st + BM * kBK + (16 * kk + tr_row) * BPITCH + wn * WN + j * 32 + tr_col;
        const u32x2 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * BPITCH);
        bfr[fs][j] = __builtin_bit_cast(bf16x8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
      } else {
        bfr[fs][j] = *reinterpret_cast<const bf16x8_t*>(&st[BM * kBK + (wn * WN + j * 32 + frag_row) * kBK + chunk]);
      }
    }
  };
  load_frags(smem, 0, 0);

  // One k-tile: four 16-wide k steps. In k step kk the wave reads the fragments of step kk+1, issues the MFMAs of
  // step kk and, interleaved with them, writes a third of the next k-tile (from a register slot) into the other
  // LDS stage and refills a quarter of that slot from global memory. The barrier sits before the last k step: by
  // then the next stage is complete and every wave has read its last fragments of the current stage, so the first
  // fragments of the next k-tile are read while the last MFMAs of this one issue.
  auto step = [&](int kt, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const uint16_t* cur = smem + (kt & 1) * STAGE;
    uint16_t* nxt = smem + ((kt + 1) & 1) * STAGE;
    const int kload = min(kt + 1 + RS, nk - 1) * kBK;  // past the end: re-reads the last k-tile (never used)
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      if (kk + 1 < kBK / 16) {
        load_frags(cur, kk + 1, (kk + 1) & 1);
      } else {
        __syncthreads();
        load_frags(nxt, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[kk & 1][j], af[kk & 1][i], acc[i][j], 0, 0, 0);
      if (kk < 3) {
#pragma unroll
        for (int c = kk * WPK; c < (kk + 1) * WPK && c < CH; ++c)
          *reinterpret_cast<u32x4*>(nxt + dst[c]) = r[slot][c];
      }
#pragma unroll
      for (int c = kk * LPK; c < (kk + 1) * LPK && c < CH; ++c) r[slot][c] = gload1(c, kload);
      // issue order: fragment reads, then MFMAs with the LDS writes and the global loads between them
      __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);
#pragma unroll
      for (int m = 0; m < NMF; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (kk < 3 && m < WPK) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        else if (m >= WPK && m < WPK + LPK) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
    }
  };
  for (int kt = 0; kt < nk; kt += RS) unroll_steps<0, RS>(step, kt);  // nk % RS == 0 (checked on the host)
  __syncthreads();

  if constexpr (PARTIAL) {  // fp32 tile -> LDS -> coalesced 16-byte row stores into ws[z]
    constexpr int FP = BN + 4;
    static_assert(BM * FP * 4 <= LDS_ELEMS * 2, "fp32 tile fits the LDS");
    float* ft = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int run = 0; run < 4; ++run) {
          const int rr = wm * WM + i * 32 + frag_row, col = wn * WN + j * 32 + 8 * run + 4 * frag_half;
          *reinterpret_cast<f32x4_t*>(&ft[rr * FP + col]) =
              f32x4_t{acc[i][j][4 * run], acc[i][j][4 * run + 1], acc[i][j][4 * run + 2], acc[i][j][4 * run + 3]};
        }
    __syncthreads();
    float* wz = g.ws + int64_t(z) * g.M * g.N;
    for (int c = tid; c < BM * (BN / 4); c += NT) {
      const int rr = c / (BN / 4), cc = (c % (BN / 4)) * 4;
      if (m0 + rr >= g.M) continue;
      store16_wt(wz + int64_t(m0 + rr) * g.N + n0 + cc, *reinterpret_cast<const u32x4*>(&ft[rr * FP + cc]));
    }
    return;
  }
  // epilogue: accumulators -> bf16 tile in LDS -> coalesced 16-byte row stores
  uint16_t* ot = smem;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int run = 0; run < 4; ++run) {
        const int rr = wm * WM + i * 32 + frag_row, col = wn * WN + j * 32 + 8 * run + 4 * frag_half;
        *reinterpret_cast<u32x2*>(&ot[rr * OUT_PITCH + col]) =
            u32x2{pack_bf16x2(acc[i][j][4 * run], acc[i][j][4 * run + 1]),
                  pack_bf16x2(acc[i][j][4 * run + 2], acc[i][j][4 * run + 3])};
      }
  __syncthreads();
  if constexpr (SILU) {  // out[m][n0/2 + j] = bf16(silu(gate) * up), gate = column j, up = column j + BN/2
    constexpr int HALF = BN / 2, CPR = HALF / 8;
    const int n2 = g.N / 2;
    for (int c = tid; c < BM * CPR; c += NT) {
      const int rr = c / CPR, cc = (c % CPR) * 8;
      const int m = m0 + rr, n = n0 / 2 + cc;
      if (m >= g.M) continue;
      const u32x4 gv = *reinterpret_cast<const u32x4*>(&ot[rr * OUT_PITCH + cc]);
      const u32x4 uv = *reinterpret_cast<const u32x4*>(&ot[rr * OUT_PITCH + HALF + cc]);
      float gf[8], uf[8], o[8];
      unpack8(gv, gf);
      unpack8(uv, uf);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = silu_bf16(gf[e]) * uf[e];
      const u32x4 v = pack8(o);
      uint16_t* d = g.c + int64_t(m) * g.scm + n;
      if (n + 8 <= n2 && (reinterpret_cast<uintptr_t>(d) & 15) == 0) {
        store16_wt(d, v);
      } else {
        for (int e = 0; e < 8 && n + e < n2; ++e) d[e] = uint16_t(v[e / 2] >> (16 * (e & 1)));
      }
    }
    return;
  }
  constexpr int CPR = BN / 8;  // 16-byte chunks per output row
  for (int c = tid; c < BM * CPR; c += NT) {
    const int rr = c / CPR, cc = (c % CPR) * 8;
    const int m = m0 + rr, n = n0 + cc;
    if (m >= g.M) continue;
    const u32x4 v = *reinterpret_cast<const u32x4*>(&ot[rr * OUT_PITCH + cc]);
    uint16_t* d = g.c + int64_t(m) * g.scm + n;
    if (n + 8 <= g.N && (reinterpret_cast<uintptr_t>(d) & 15) == 0) {
      store16_wt(d, v);
    } else {
      for (int e = 0; e < 8 && n + e < g.N; ++e) d[e] = uint16_t(v[e / 2] >> (16 * (e & 1)));
    }
  }
}

// ------------------------------------------------------------------------------------------------------------
// Skinny bf16 kernel for M <= 32 (decode batches), bound by reading W once: a block owns 16 output columns for all
// M rows and its NW waves split K between them (wave w takes the 32-wide k steps w, w + NW, ..., so the block's
// loads in flight cover NW consecutive steps of each W row). Each wave multiplies with v_mfma_f32_16x16x32_bf16
// fed straight from global memory (lane l: row l % 16, k = 8 * (l / 16) .. +8 of the step, for both the A rows
// and the W rows; W is read once, A is small and stays in L2), U steps of loads issued before their MFMAs. The
// NW partial 16-row tiles are summed through LDS in wave order (deterministic), rounded to bf16 and stored.

// SILU: W = [gate; up] ([2 * N2, K], N = 2 * N2), C [M, N2]: the block takes gate rows n0 .. and up rows N2 + n0 ..
// and stores bf16(silu(gate) * up) of the two rounded sums (bitwise the unfused result).
template <int MT, int NCOL, int NW, int U, bool SILU = false>
__global__ __launch_bounds__(NW * 64) void gemm_skinny(const MfmaArgs g) {
  constexpr int NP = SILU ? 2 : 1;              // products per block: (gate, up) or the plain one
  constexpr int NT = NCOL >= 16 ? NCOL / 16 : 1;  // 16-column MFMA tiles per block (they share the A fragments)
  static_assert(NCOL == 8 || NCOL == 16 || NCOL == 32 || NCOL == 64, "output columns per block");
  __shared__ float red[NW][NP][NT][MT][4][64];
  const int n0 = blockIdx.x * NCOL, m0 = blockIdx.y * 16 * MT;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int fr = lane % 16, fk = (lane / 16) * 8;
  const int nout = SILU ? g.N / 2 : g.N;
  // with NCOL = 8 the MFMA's columns 8..15 repeat columns 0..7 (same addresses, merged by the memory pipeline)
  const uint16_t* wrows[NP][NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int wn = min(n0 + 16 * j + (NCOL == 8 ? fr % 8 : fr), nout - 1);
    wrows[0][j] = g.w + int64_t(wn) * g.swn + fk;
    if constexpr (SILU) wrows[NP - 1][j] = g.w + int64_t(nout + wn) * g.swn + fk;
  }
  const uint16_t* arow[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) arow[t] = g.a + int64_t(min(m0 + t * 16 + fr, g.M - 1)) * g.sam + fk;
  f32x4_t acc[NP][NT][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[p][j][t] = f32x4_t{};
  const int nks = (g.K + 31) / 32;
  for (int s0 = wave; s0 < nks; s0 += NW * U) {
    bf16x8_t wf[U][NP][NT], af[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ks = s0 + u * NW, k = ks * 32;
      const bool in = ks < nks && k + fk < g.K;  // K % 8 == 0: a lane's 8 values are all in or all out
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          wf[u][p][j] = in ? *reinterpret_cast<const bf16x8_t*>(wrows[p][j] + k) : bf16x8_t{};
#pragma unroll
      for (int t = 0; t < MT; ++t) af[u][t] = in ? *reinterpret_cast<const bf16x8_t*>(arow[t] + k) : bf16x8_t{};
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int t = 0; t < MT; ++t)
            acc[p][j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[u][t], wf[u][p][j], acc[p][j][t], 0, 0, 0);
  }
  // lane l, register r of tile (j, t) holds C row m0 + t*16 + 4*(l/16) + r, column n0 + 16 j + l%16
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][p][j][t][r][lane] = acc[p][j][t][r];
  __syncthreads();
  for (int idx = threadIdx.x; idx < NT * MT * 256; idx += NW * 64) {
    const int j = idx / (MT * 256), t = (idx / 256) % MT, r = (idx / 64) % 4, l = idx % 64;
    float sum[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      sum[p] = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum[p] += red[w][p][j][t][r][l];
    }
    const int m = m0 + t * 16 + 4 * (l / 16) + r, n = n0 + 16 * j + l % 16;
    if ((NCOL == 8 && l % 16 >= 8) || m >= g.M || n >= nout) continue;
    float o = sum[0];
    if constexpr (SILU) o = silu_bf16(round_bf16(sum[0])) * round_bf16(sum[1]);
    g.c[int64_t(m) * g.scm + n] = f32_to_bf16(o);
  }
}

// gemm_skinny with the operands staged through LDS: the same k steps per wave in the same order and the same MFMA
// operands (so the same bits), but a round of KR = NW * UR * 32 consecutive k of the block's A rows and W rows is
// loaded by the whole block with 16-byte loads that run along the rows (32 lanes cover 512 contiguous bytes), and
// each wave then reads its fragments from LDS. Read straight from memory, a fragment load touches 16 rows x 64 bytes
// per wave instruction and streams ~31-36 GB/s per CU from L2; row-contiguous loads of the same bytes 55-75 GB/s.
// Two LDS stages (round r + 1 stored while round r is multiplied, round r + 2 in flight in registers); row pitch
// KR + 8 elements. Past K the staged chunks are zero, as gemm_skinny's loads are. ONE (K <= KR): the whole K in one
// round and one stage, every load of the block in flight at once (one memory round trip instead of one per round).
template <int MT, int NCOL, int NW, int UR, bool SILU = false, bool ONE = false>
__global__ __launch_bounds__(NW * 64) void gemm_skinny_lds(const MfmaArgs g) {
  constexpr int NP = SILU ? 2 : 1;
  constexpr int NT = NCOL >= 16 ? NCOL / 16 : 1;
  static_assert(NCOL == 8 || NCOL == 16 || NCOL == 32 || NCOL == 64, "output columns per block");
  constexpr int RA = 16 * MT, RW = NP * NCOL;  // staged rows: A rows, then W rows (product p, column j)
  constexpr int KR = NW * UR * 32, PITCH = KR + 8, CPR = KR / 8;
  constexpr int NTH = NW * 64, NCH = (RA + RW) * CPR, CPT = (NCH + NTH - 1) / NTH;
  constexpr int STAGE = (RA + RW) * PITCH;  // bf16 elements
  constexpr int RED = NW * NP * NT * MT * 4 * 64;  // floats of the cross-wave reduction (after the last round)
  constexpr int LDS_BYTES = (ONE ? 2 : 4) * STAGE > 4 * RED ? (ONE ? 2 : 4) * STAGE : 4 * RED;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  uint16_t* st = reinterpret_cast<uint16_t*>(lds);
  const int n0 = blockIdx.x * NCOL, m0 = blockIdx.y * RA;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int fr = lane % 16, fk = (lane / 16) * 8;
  const int nout = SILU ? g.N / 2 : g.N;

  // chunk c = tid + NTH * i of a round: staged row c / CPR, 16-byte chunk c % CPR of it
  const uint16_t* src[CPT];
  int dst[CPT], kof[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = min(tid + NTH * i, NCH - 1), r = c / CPR, kc = c % CPR;
    if (r < RA) {
      src[i] = g.a + int64_t(min(m0 + r, g.M - 1)) * g.sam + kc * 8;
    } else {
      const int p = (r - RA) / NCOL, j = (r - RA) % NCOL;
      src[i] = g.w + int64_t(p * nout + min(n0 + j, nout - 1)) * g.swn + kc * 8;
    }
    dst[i] = r * PITCH + kc * 8;
    kof[i] = kc * 8;
  }
  auto live = [&](int i) { return NCH % NTH == 0 || i + 1 < CPT || tid + NTH * i < NCH; };
  u32x4 v[CPT];
  auto load_round = [&](int r) {
    const int k0 = r * KR;
    // W rows (staged rows RA ..) are read once per launch: the nontemporal hint; the A rows, which every block
    // reads, stay cached
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const u32x4* p = reinterpret_cast<const u32x4*>(src[i] + k0);
      const bool w_row = min(tid + NTH * i, NCH - 1) / CPR >= RA;
      v[i] = (live(i) && k0 + kof[i] < g.K) ? (w_row ? __builtin_nontemporal_load(p) : *p) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_round = [&](int stage) {
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      if (live(i)) *reinterpret_cast<u32x4*>(st + stage * STAGE + dst[i]) = v[i];
  };

  f32x4_t acc[NP][NT][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[p][j][t] = f32x4_t{};
  const int rounds = ONE ? 1 : (g.K + KR - 1) / KR;
  load_round(0);
  store_round(0);
  if (!ONE && rounds > 1) load_round(1);
  __syncthreads();
  for (int r = 0; r < rounds; ++r) {
    const uint16_t* s = st + (r & 1) * STAGE;
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int kl = (wave + NW * u) * 32 + fk;  // the wave's k step wave + NW (r UR + u), this lane's 8 k
      bf16x8_t af[MT], wf[NP][NT];
#pragma unroll
      for (int t = 0; t < MT; ++t) af[t] = *reinterpret_cast<const bf16x8_t*>(s + (16 * t + fr) * PITCH + kl);
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int col = NCOL == 8 ? fr % 8 : 16 * j + fr;  // 8 columns: MFMA columns 8..15 repeat 0..7
          wf[p][j] = *reinterpret_cast<const bf16x8_t*>(s + (RA + p * NCOL + col) * PITCH + kl);
        }
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int t = 0; t < MT; ++t)
            acc[p][j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t], wf[p][j], acc[p][j][t], 0, 0, 0);
    }
    if (!ONE && r + 1 < rounds) {
      store_round((r + 1) & 1);
      if (r + 2 < rounds) load_round(r + 2);
    }
    __syncthreads();
  }
  // cross-wave sum in wave order (the LDS of the stages, no longer read), as gemm_skinny
  float* red = reinterpret_cast<float*>(lds);
  auto ridx = [&](int w, int p, int j, int t, int rr, int l) {
    return ((((w * NP + p) * NT + j) * MT + t) * 4 + rr) * 64 + l;
  };
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) red[ridx(wave, p, j, t, rr, lane)] = acc[p][j][t][rr];
  __syncthreads();
  for (int idx = tid; idx < NT * MT * 256; idx += NTH) {
    const int j = idx / (MT * 256), t = (idx / 256) % MT, rr = (idx / 64) % 4, l = idx % 64;
    float sum[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      sum[p] = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum[p] += red[ridx(w, p, j, t, rr, l)];
    }
    const int m = m0 + t * 16 + 4 * (l / 16) + rr, n = n0 + 16 * j + l % 16;
    if ((NCOL == 8 && l % 16 >= 8) || m >= g.M || n >= nout) continue;
    float o = sum[0];
    if constexpr (SILU) o = silu_bf16(round_bf16(sum[0])) * round_bf16(sum[1]);
    g.c[int64_t(m) * g.scm + n] = f32_to_bf16(o);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Wide decode outputs with K = 1024 (the tied LM head: 32 x 151 936 x 1024, a 311 MB weight): the block stages its
// A rows (all M <= 32 of them, the whole K) in LDS once, and wave gw of the grid's nw takes the 16-column W tiles
// gw, gw + nw, ... (neighbouring waves read neighbouring tiles), v_mfma_f32_16x16x32_bf16 with the 32 k steps of a
// tile accumulated in k order (no cross-wave sum), A fragments read from LDS four k steps at a time. Each wave
// stages its tiles through its own LDS slice: a tile's 16 rows come in quarters of K (16 rows x 256 k, 8 KB) loaded
// along the rows (two rows of 512 contiguous bytes per instruction) with the nontemporal hint, two quarters in
// flight in registers while the wave multiplies the quarter in its slice. 151 936 x 1024 at M = 32, the weight from
// HBM: 57.3 us against 63.6 us with the W fragments loaded straight from memory (16 rows x 64 bytes per
// instruction, half a 128-byte line each; the same MFMAs in the same order, so the same bits); staged with plain
// loads 65.8 us, three quarters in flight 57.5 us. Earlier variants of the fragment loads: 64-column LDS-staged
// blocks (gemm_skinny_lds) 67.1 us, a contiguous range of tiles per wave 67.6 us, nontemporal fragment loads
// 71.0 us, the A fragments kept in registers (one wave per SIMD) 73.2 us.
template <int MT>
__global__ __launch_bounds__(512) void gemm_wide_k1024(const MfmaArgs g) {
  constexpr int DEPTH = 2;  // quarters in flight
  constexpr int K = 1024, P = K + 8, Q = 256, QP = Q + 8, NQ = K / Q;
  __shared__ __attribute__((aligned(16))) uint16_t As[16 * MT * P];
  __shared__ __attribute__((aligned(16))) uint16_t Wsl[8 * 16 * QP];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  for (int c = threadIdx.x; c < 16 * MT * (K / 8); c += 512) {
    const int r = c / (K / 8), k = (c % (K / 8)) * 8;
    *reinterpret_cast<u32x4*>(As + r * P + k) =
        *reinterpret_cast<const u32x4*>(g.a + int64_t(min(r, g.M - 1)) * g.sam + k);
  }
  __syncthreads();  // the last block-wide step: the waves run on their own from here
  const int nw = gridDim.x * 8, ntiles = (g.N + 15) / 16, tile0 = blockIdx.x * 8 + wave;
  if (tile0 >= ntiles) return;
  const int nunits = ((ntiles - 1 - tile0) / nw + 1) * NQ;  // (tile, quarter) units of this wave
  const int fr = lane % 16, fk = (lane / 16) * 8;
  uint16_t* ws = Wsl + wave * 16 * QP;
  // unit u: tile tile0 + (u / NQ) nw, quarter u % NQ; instruction i loads rows 2 i + lane / 32, chunk lane % 32
  auto qload = [&](u32x4 (&r)[8], int u) {
    const int tile = tile0 + (u / NQ) * nw, q = u % NQ;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int n = min(16 * tile + 2 * i + lane / 32, g.N - 1);
      const u32x4* p = reinterpret_cast<const u32x4*>(g.w + int64_t(n) * g.swn + q * Q + (lane % 32) * 8);
      r[i] = __builtin_nontemporal_load(p);  // read once
    }
  };
  f32x4_t acc[MT];
  auto unit = [&](u32x4 (&r)[8], int u) {
    const int tile = tile0 + (u / NQ) * nw, q = u % NQ;
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(ws + (2 * i + lane / 32) * QP + (lane % 32) * 8) = r[i];
    if (u + DEPTH < nunits) qload(r, u + DEPTH);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (q == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{};
    }
#pragma unroll
    for (int k4 = 0; k4 < Q / 32; k4 += 4) {
      bf16x8_t av[4][MT], wv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wv[k] = *reinterpret_cast<const bf16x8_t*>(ws + fr * QP + 32 * (k4 + k) + fk);
#pragma unroll
        for (int t = 0; t < MT; ++t)
          av[k][t] = *reinterpret_cast<const bf16x8_t*>(As + (16 * t + fr) * P + q * Q + 32 * (k4 + k) + fk);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[k][t], wv[k], acc[t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    // every lane has its fragments of this quarter (the MFMAs consumed them) before the slice is written again
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (q == NQ - 1) {  // lane l, register r of row tile t holds C row 16 t + 4 (l / 16) + r, column 16 tile + l % 16
      const int n = 16 * tile + fr;
      if (n < g.N) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int m = 16 * t + 4 * (lane / 16) + rr;
            if (m < g.M) g.c[int64_t(m) * g.scm + n] = f32_to_bf16(acc[t][rr]);
          }
      }
    }
  };
  u32x4 r0[8], r1[8];
  qload(r0, 0);
  if (nunits > 1) qload(r1, 1);
  for (int u = 0; u < nunits; u += DEPTH) {
    unit(r0, u);
    if (u + 1 < nunits) unit(r1, u + 1);
  }
}

// ------------------------------------------------------------------------------------------------------------
// RMSNorm (or Add+RMSNorm) of the A rows fused into the decode GEMM (M <= 32): the norm that precedes a projection
// (input_layernorm -> qkv, post_attention_layernorm -> gate_up) in the same launch. Every block normalises the
// 16 * MT rows it multiplies -- K = 256 * KC, half a wave per row, each lane the same KC 16-byte chunks and the
// same fp32 order as norm_kernel<32, KC, ADD> (rms_norm.hip, torch's order for M rows), so the normalised bf16
// values are bitwise that kernel's output -- into LDS, and the blocks of the first column tile also write the
// residual sum. The block's W fragments (one round: K / 32 k steps over NW waves x U) are requested right after the
// rows, so the norm runs while they are in flight; the A fragments then come from LDS. The per-column k order is
// that of gemm_skinny, so the product is bitwise the two-launch result (norm, then matmul / matmul_silu_mul).
struct NormMfmaArgs {
  MfmaArgs g;              // g.a is not used: A = norm(x [+ r])
  const uint16_t* x;       // [M, K], row stride sx
  const uint16_t* r;       // residual [M, K], row stride sr (ADD)
  const uint16_t* nw;      // norm weight [K]
  uint16_t* res_out;       // [M, K] contiguous: bf16(x + r) (ADD)
  int64_t sx, sr;
  float factor, eps;       // the mean's factor for M rows (aten_mean_factor) and epsilon
  int m;                   // aten_norm_bw(K, M) / 64
};

template <int MT, int NCOL, bool SILU, int KC, bool ADD>
__global__ __launch_bounds__(512) void gemm_skinny_norm(const NormMfmaArgs a) {
  constexpr int NW = 8;
  constexpr int K = 256 * KC, KP = K + 8;  // LDS row pitch: the 16 rows of a fragment read hit distinct banks
  constexpr int U = K / 32 / NW;               // k steps per wave: the whole K in one round
  constexpr int R = 16 * MT;                   // rows of this block
  constexpr int NP = SILU ? 2 : 1;
  constexpr int NT = NCOL >= 16 ? NCOL / 16 : 1;
  static_assert(NCOL == 8 || NCOL == 16 || NCOL == 32, "output columns per block");
  static_assert(U >= 1 && U * 32 * NW == K, "one round of k steps");
  // LDS: the normalised rows, then the block's W rows (staged with row-contiguous loads), whose bytes the
  // cross-wave reduction reuses once every wave has read its W fragments
  // (when they fit: not the K = 2048 tiles, which read their W fragments straight from memory)
  constexpr int RW = NP * NCOL;                  // staged W rows: product p, column c at row p * NCOL + c
  constexpr int WCH = RW * (K / 8), WCT = (WCH + 511) / 512;  // 16-byte W chunks, per thread
  static_assert(WCH % 512 == 0, "whole W chunks per thread");
  constexpr int A_BYTES = R * KP * 2, RED_BYTES = NW * NP * NT * MT * 4 * 64 * 4;
  constexpr bool STAGE_W = A_BYTES + RW * KP * 2 <= 160 * 1024;
  constexpr int W_BYTES = STAGE_W ? RW * KP * 2 : 0;
  __shared__ __attribute__((aligned(16))) unsigned char lds[A_BYTES + (W_BYTES > RED_BYTES ? W_BYTES : RED_BYTES)];
  uint16_t* As = reinterpret_cast<uint16_t*>(lds);
  uint16_t* Ws = reinterpret_cast<uint16_t*>(lds + A_BYTES);
  auto red = reinterpret_cast<float (*)[NP][NT][MT][4][64]>(lds + A_BYTES);
  const MfmaArgs& g = a.g;
  const int n0 = blockIdx.x * NCOL, m0 = blockIdx.y * R;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int fr = lane % 16, fk = (lane / 16) * 8;
  const int nout = SILU ? g.N / 2 : g.N;

  u32x4 wst[STAGE_W ? WCT : 1];  // STAGE_W: this thread's W chunks, chunk c = tid + 512 i, staged row c / (K / 8)
  bf16x8_t wfd[STAGE_W ? 1 : U][NP][NT];  // else the W fragments of the whole K (wave w: k steps w, w + NW, ...)

  // the block's rows, normalised, into LDS: half h = lane / 32 of wave w takes rows w + (2 i + h) NW, lane
  // j = lane % 32 the chunks at elements 8 j + 256 k (rows past M are computed from row M - 1 and stored as zeros,
  // so no lane leaves the reduction). All of the wave's row loads are issued before the first store: the
  // new-residual stores could alias the next rows' inputs for all the compiler knows, so loads written after them
  // would have to wait for them.
  constexpr int RH = R / NW / 2;  // rows per half-wave
  static_assert(RH * 2 * NW == R, "whole row pairs per wave");
  const int half = lane / 32, cj = (lane % 32) * 8;
  u32x4 raw[RH][KC], rraw[RH][KC], wraw[KC];
#pragma unroll
  for (int i = 0; i < RH; ++i) {
    const int m = min(m0 + wave + (2 * i + half) * NW, g.M - 1);
#pragma unroll
    for (int k = 0; k < KC; ++k) raw[i][k] = load8<true>(a.x + int64_t(m) * a.sx + 256 * k + cj);
    if constexpr (ADD)
#pragma unroll
      for (int k = 0; k < KC; ++k) rraw[i][k] = load8<true>(a.r + int64_t(m) * a.sr + 256 * k + cj);
  }
#pragma unroll
  for (int k = 0; k < KC; ++k) wraw[k] = load8<true>(a.nw + 256 * k + cj);
  // then the W rows: loads return in issue order, so the rows' loads come in first and the norm below runs while
  // the weight is still on its way from HBM (issued the other way round, every row load waited for the weight's:
  // qkv + Add+RMSNorm at M = 32 6.66 -> 6.37 us, gate_up + SiLU 8.44 -> 8.06 us). 16-byte loads along the rows (32
  // lanes cover 512 contiguous bytes) into LDS, not fragments straight from memory (16 rows x 64 bytes per
  // instruction, half a 128-byte line each).
  if constexpr (STAGE_W) {
#pragma unroll
    for (int i = 0; i < WCT; ++i) {
      const int c = threadIdx.x + 512 * i, row = c / (K / 8), p = row / NCOL, wn = min(n0 + row % NCOL, nout - 1);
      // read once per launch: the nontemporal hint (decode step 1712 -> 1692 us with the hint here and on the W rows
      // of gemm_skinny_lds; alone, the launches time the same either way)
      const uint16_t* wp = g.w + int64_t(p == 0 ? wn : nout + wn) * g.swn + (c % (K / 8)) * 8;
      wst[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp));
    }
  } else {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int wn = min(n0 + 16 * j + (NCOL == 8 ? fr % 8 : fr), nout - 1);
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const uint16_t* wrow = g.w + int64_t(p == 0 ? wn : nout + wn) * g.swn + fk;
#pragma unroll
        for (int u = 0; u < U; ++u) wfd[u][p][j] = *reinterpret_cast<const bf16x8_t*>(wrow + (wave + u * NW) * 32);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RH; ++i) {
    const int rl = wave + (2 * i + half) * NW, m = m0 + rl;
    uint16_t* dst = As + rl * KP;
    float v[KC][8];
    if constexpr (ADD) {
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        float xf[8], rf[8];
        unpack8(raw[i][k], xf);
        unpack8(rraw[i][k], rf);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = xf[e] + rf[e];
        if (blockIdx.x == 0 && m < g.M) store8<true>(a.res_out + int64_t(m) * K + 256 * k + cj, pack8(v[k]));
      }
    } else {
#pragma unroll
      for (int k = 0; k < KC; ++k) unpack8(raw[i][k], v[k]);
    }
    const float rstd = torch_rsqrt(group_sum<32>(t32_partial_m<KC>(v, a.m)) * a.factor + a.eps);
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      float wfl[8], o[8];
      unpack8(wraw[k], wfl);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = round_bf16(v[k][e] * rstd) * wfl[e];
      *reinterpret_cast<u32x4*>(dst + 256 * k + cj) = m < g.M ? pack8(o) : u32x4{0, 0, 0, 0};
    }
  }
  if constexpr (STAGE_W) {
#pragma unroll
    for (int i = 0; i < WCT; ++i) {
      const int c = threadIdx.x + 512 * i;
      *reinterpret_cast<u32x4*>(Ws + (c / (K / 8)) * KP + (c % (K / 8)) * 8) = wst[i];
    }
  }
  __syncthreads();

  f32x4_t acc[NP][NT][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[p][j][t] = f32x4_t{};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int k = (wave + u * NW) * 32;
    bf16x8_t af[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) af[t] = *reinterpret_cast<const bf16x8_t*>(As + (t * 16 + fr) * KP + k + fk);
    bf16x8_t wf[NP][NT];  // with NCOL = 8 the MFMA's columns 8..15 repeat columns 0..7
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if constexpr (STAGE_W)
          wf[p][j] = *reinterpret_cast<const bf16x8_t*>(Ws + (p * NCOL + (NCOL == 8 ? fr % 8 : 16 * j + fr)) * KP +
                                                         k + fk);
        else
          wf[p][j] = wfd[u][p][j];
      }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          acc[p][j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t], wf[p][j], acc[p][j][t], 0, 0, 0);
  }
  if constexpr (STAGE_W) __syncthreads();  // every wave has read its W fragments: the reduction reuses their bytes
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][p][j][t][r][lane] = acc[p][j][t][r];
  __syncthreads();
  for (int idx = threadIdx.x; idx < NT * MT * 256; idx += NW * 64) {
    const int j = idx / (MT * 256), t = (idx / 256) % MT, r = (idx / 64) % 4, l = idx % 64;
    float sum[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      sum[p] = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum[p] += red[w][p][j][t][r][l];
    }
    const int m = m0 + t * 16 + 4 * (l / 16) + r, n = n0 + 16 * j + l % 16;
    if ((NCOL == 8 && l % 16 >= 8) || m >= g.M || n >= nout) continue;
    float o = sum[0];
    if constexpr (SILU) o = silu_bf16(round_bf16(sum[0])) * round_bf16(sum[1]);
    g.c[int64_t(m) * g.scm + n] = f32_to_bf16(o);
  }
}

// ------------------------------------------------------------------------------------------------------------
// fp32 MFMA kernel: v_mfma_f32_32x32x2_f32 forms exact fp32 products and accumulates them in fp32 (precision
// "ieee"); with TF32 every input is first rounded to tf32. A is K-contiguous; B is either K-contiguous (W [N, K],
// B = W.t()) or N-contiguous ([K, N]). BM x BN block tile of WAVES_M x WAVES_N waves, each owning (BM / WAVES_M) x
// (BN / WAVES_N) outputs as 32x32 MFMA tiles (operands swapped as in the bf16 kernel), k-tile 32. LDS holds both
// operands k-major ([k][m], [k][n]) with row pitches of BM + 32 and BN + 32 floats (32 mod 64 banks), so the two
// half-waves of a fragment read (rows k and k+1, 32 consecutive floats each) hit disjoint bank halves. Global loads
// are 16 bytes: 4 consecutive k of one row of A / W (8 lanes cover one row's 128 bytes), or 4 consecutive n of one
// row of B. The next k-tile is loaded into registers at the start of the current one and stored into the other LDS
// stage halfway through its MFMAs (stores after the last MFMA left the matrix cores idle during them). 4096^3:
// 256x256 tiles with 16 waves (4 per SIMD) 1107 us, 128x128 with 8 waves 1167 us, 128x128 with 4 waves and the
// stores at the end 1434 us.
struct F32Args {
  float* c;
  const float* a;
  const float* b;
  int M, N, K;
  int64_t sam, sbk, sbn, scm;
};

template <int BM, int BN, int WAVES_M, int WAVES_N, bool B_NMAJOR, bool TF32>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_mfma_f32(const F32Args g) {
  constexpr int NT = 64 * WAVES_M * WAVES_N, BK = 32, PA = BM + 32, PB = BN + 32;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N, FM = WM / 32, FN = WN / 32;
  constexpr int CHA = BM * BK / 4 / NT, CHB = BN * BK / 4 / NT;  // 16-byte chunks per thread per k-tile
  static_assert(FM >= 1 && FN >= 1 && CHA >= 1 && CHB >= 1 && CHA * NT * 4 == BM * BK && CHB * NT * 4 == BN * BK,
                "tile shape");
  __shared__ __attribute__((aligned(16))) float lds[2][BK * (PA + PB)];  // [stage][A k-major | B k-major]
  int pid_m, pid_n;
  tile_coords(blockIdx.x, g.M, g.N, BM, BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // K-major chunks (A, and B when K-contiguous): chunk c covers row c / 8, k = 4 * (c % 8) .. +4
  const float* asrc[CHA];
  const float* bsrc[CHB];
  int arow[CHA], akc[CHA], brow[CHB], bkc[CHB];
#pragma unroll
  for (int i = 0; i < CHA; ++i) {
    const int c = tid + NT * i;
    arow[i] = c / 8;
    akc[i] = 4 * (c % 8);
    asrc[i] = g.a + int64_t(min(m0 + arow[i], g.M - 1)) * g.sam + akc[i];
  }
#pragma unroll
  for (int i = 0; i < CHB; ++i) {
    const int c = tid + NT * i;
    if constexpr (B_NMAJOR) {  // chunk c covers k row c / (BN / 4), n = 4 * (c % (BN / 4)) .. +4 (clamped inside N)
      brow[i] = c / (BN / 4);
      bkc[i] = 4 * (c % (BN / 4));
      bsrc[i] = g.b + min(n0 + bkc[i], g.N - 4);
    } else {
      brow[i] = c / 8;
      bkc[i] = 4 * (c % 8);
      bsrc[i] = g.b + int64_t(min(n0 + brow[i], g.N - 1)) * g.sbn + bkc[i];
    }
  }
  f32x4_t ra[CHA], rb[CHB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CHA; ++i)
      ra[i] = (k0 + akc[i] < g.K) ? *reinterpret_cast<const f32x4_t*>(asrc[i] + k0) : f32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < CHB; ++i) {
      if constexpr (B_NMAJOR)
        rb[i] = (k0 + brow[i] < g.K) ? *reinterpret_cast<const f32x4_t*>(bsrc[i] + int64_t(k0 + brow[i]) * g.sbk)
                                     : f32x4_t{0, 0, 0, 0};
      else
        rb[i] = (k0 + bkc[i] < g.K) ? *reinterpret_cast<const f32x4_t*>(bsrc[i] + k0) : f32x4_t{0, 0, 0, 0};
    }
  };
  auto tf = [](float x) { return TF32 ? round_tf32(x) : x; };
  auto lstore = [&](int st) {
    float* la = lds[st];
    float* lb = lds[st] + BK * PA;
#pragma unroll
    for (int i = 0; i < CHA; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) la[(akc[i] + e) * PA + arow[i]] = tf(ra[i][e]);
#pragma unroll
    for (int i = 0; i < CHB; ++i) {
      if constexpr (B_NMAJOR) {
        *reinterpret_cast<f32x4_t*>(&lb[brow[i] * PB + bkc[i]]) =
            f32x4_t{tf(rb[i][0]), tf(rb[i][1]), tf(rb[i][2]), tf(rb[i][3])};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) lb[(bkc[i] + e) * PB + brow[i]] = tf(rb[i][e]);
      }
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16_t{};
  const int fr = lane % 32, fk = lane / 32;
  const int nk = (g.K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) gload((kt + 1) * BK);
    const float* la = lds[kt & 1];
    const float* lb = lds[kt & 1] + BK * PA;
#pragma unroll
    for (int kp = 0; kp < BK / 2; ++kp) {
      float af[FM], bfv[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = la[(2 * kp + fk) * PA + wm * WM + i * 32 + fr];
#pragma unroll
      for (int j = 0; j < FN; ++j) bfv[j] = lb[(2 * kp + fk) * PB + wn * WN + j * 32 + fr];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bfv[j], af[i], acc[i][j], 0, 0, 0);
      if (kp == BK / 4 - 1 && more) lstore((kt + 1) & 1);  // the other stage: nobody reads it during this k-tile
    }
    __syncthreads();
  }
  // lane holds C row m0 + wm*WM + i*32 + lane%32, columns n0 + wn*WN + j*32 + 8*q + 4*(lane/32) .. +4
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * WM + i * 32 + fr;
    if (m >= g.M) continue;
    float* crow = g.c + int64_t(m) * g.scm;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WN + j * 32 + 8 * q + 4 * fk;
        const f32x4_t v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        if (n + 4 <= g.N && (reinterpret_cast<uintptr_t>(crow + n) & 15) == 0) {
          *reinterpret_cast<f32x4_t*>(crow + n) = v;
        } else {
          for (int e = 0; e < 4 && n + e < g.N; ++e) crow[n + e] = v[e];
        }
      }
  }
}

// fp32 MFMA GEMM reading its fragments 16 bytes at a time: both operands sit in LDS as k-contiguous rows (A as it
// lies; a K-contiguous B as it lies, an N-contiguous B transposed while it is staged), row pitch BK + 4 floats (the
// 16 rows of a quarter-wave's 16-byte reads fall on distinct banks). The k-tile of 32 is taken in 4 groups of 8 k:
// lane l (row or column l % 32, half h = l / 32) reads k = 8 g + 4 h .. +4 of group g in one ds_read_b128, and MFMA
// step s of the group uses its element s -- k = 8 g + s for half 0 and 8 g + 4 + s for half 1 -- so 4 MFMA steps
// take one read per fragment instead of four. (The products are summed in that k order.) The next group's
// fragments are read while the current group's MFMAs issue; the next k-tile is loaded into registers at the start
// of a k-tile and stored into the other LDS stage after its second group.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool B_NMAJOR, bool TF32, bool PF = true>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_mfma_f32q(const F32Args g) {
  constexpr int NT = 64 * WAVES_M * WAVES_N, BK = 32, P = BK + 4;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N, FM = WM / 32, FN = WN / 32;
  constexpr int CHA = BM * BK / 4 / NT, CHB = BN * BK / 4 / NT;  // 16-byte chunks per thread per k-tile
  static_assert(FM >= 1 && FN >= 1 && CHA >= 1 && CHB >= 1 && CHA * NT * 4 == BM * BK && CHB * NT * 4 == BN * BK,
                "tile shape");
  static_assert(!B_NMAJOR || (BN % 32 == 0 && BK % 8 == 0), "N-contiguous B staging");
  __shared__ __attribute__((aligned(16))) float lds[2][(BM + BN) * P];  // [stage][A rows | B rows]
  int pid_m, pid_n;
  tile_coords(blockIdx.x, g.M, g.N, BM, BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // A (and a K-contiguous B) chunk c: row c / 8, k 4 (c % 8) .. +4. N-contiguous B chunk c: k row kk, columns
  // 4 nn .. +4 with 8 lanes along n (128 contiguous bytes) and 8 along k
  const float* asrc[CHA];
  const float* bsrc[CHB];
  int adst[CHA], akc[CHA], bdst[CHB], bkc[CHB];
#pragma unroll
  for (int i = 0; i < CHA; ++i) {
    const int c = tid + NT * i, row = c / 8;
    akc[i] = 4 * (c % 8);
    asrc[i] = g.a + int64_t(min(m0 + row, g.M - 1)) * g.sam + akc[i];
    adst[i] = row * P + akc[i];
  }
#pragma unroll
  for (int i = 0; i < CHB; ++i) {
    const int c = tid + NT * i;
    if constexpr (B_NMAJOR) {
      constexpr int NH = BN / 32;  // groups of 8 column chunks
      const int nn = ((c / 64) % NH) * 8 + c % 8, kk = (c / (64 * NH)) * 8 + (c / 8) % 8;
      bkc[i] = kk;
      bsrc[i] = g.b + min(n0 + 4 * nn, g.N - 4);
      bdst[i] = BM * P + 4 * nn * P + kk;
    } else {
      const int row = c / 8;
      bkc[i] = 4 * (c % 8);
      bsrc[i] = g.b + int64_t(min(n0 + row, g.N - 1)) * g.sbn + bkc[i];
      bdst[i] = BM * P + row * P + bkc[i];
    }
  }
  f32x4_t ra[CHA], rb[CHB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CHA; ++i)
      ra[i] = (k0 + akc[i] < g.K) ? *reinterpret_cast<const f32x4_t*>(asrc[i] + k0) : f32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < CHB; ++i) {
      if constexpr (B_NMAJOR)
        rb[i] = (k0 + bkc[i] < g.K) ? *reinterpret_cast<const f32x4_t*>(bsrc[i] + int64_t(k0 + bkc[i]) * g.sbk)
                                    : f32x4_t{0, 0, 0, 0};
      else
        rb[i] = (k0 + bkc[i] < g.K) ? *reinterpret_cast<const f32x4_t*>(bsrc[i] + k0) : f32x4_t{0, 0, 0, 0};
    }
  };
  auto tf = [](float x) { return TF32 ? round_tf32(x) : x; };
  auto lstore = [&](int st) {
    float* l = lds[st];
#pragma unroll
    for (int i = 0; i < CHA; ++i)
      *reinterpret_cast<f32x4_t*>(l + adst[i]) = f32x4_t{tf(ra[i][0]), tf(ra[i][1]), tf(ra[i][2]), tf(ra[i][3])};
#pragma unroll
    for (int i = 0; i < CHB; ++i) {
      if constexpr (B_NMAJOR) {
#pragma unroll
        for (int e = 0; e < 4; ++e) l[bdst[i] + e * P] = tf(rb[i][e]);
      } else {
        *reinterpret_cast<f32x4_t*>(l + bdst[i]) = f32x4_t{tf(rb[i][0]), tf(rb[i][1]), tf(rb[i][2]), tf(rb[i][3])};
      }
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16_t{};
  const int fr = lane % 32, fh = lane / 32;
  const int nk = (g.K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) gload((kt + 1) * BK);
    const float* la = lds[kt & 1];
    const float* lb = lds[kt & 1] + BM * P;
    f32x4_t af[2][FM], bf[2][FN];  // fragments of group q and q + 1
    auto frags = [&](int q, int sl) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[sl][i] = *reinterpret_cast<const f32x4_t*>(la + (wm * WM + i * 32 + fr) * P + 8 * q + 4 * fh);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[sl][j] = *reinterpret_cast<const f32x4_t*>(lb + (wn * WN + j * 32 + fr) * P + 8 * q + 4 * fh);
    };
    if (PF) frags(0, 0);
#pragma unroll
    for (int q = 0; q < BK / 8; ++q) {
      if (PF && q + 1 < BK / 8) frags(q + 1, (q + 1) & 1);
      if (!PF) frags(q, q & 1);
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[q & 1][j][st], af[q & 1][i][st], acc[i][j], 0, 0, 0);
      if (q == 1 && more) lstore((kt + 1) & 1);  // the other stage: nobody reads it during this k-tile
    }
    __syncthreads();
  }
  // lane holds C row m0 + wm*WM + i*32 + lane%32, columns n0 + wn*WN + j*32 + 8*q + 4*(lane/32) .. +4
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * WM + i * 32 + fr;
    if (m >= g.M) continue;
    float* crow = g.c + int64_t(m) * g.scm;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WN + j * 32 + 8 * q + 4 * fh;
        const f32x4_t v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        if (n + 4 <= g.N && (reinterpret_cast<uintptr_t>(crow + n) & 15) == 0) {
          *reinterpret_cast<f32x4_t*>(crow + n) = v;
        } else {
          for (int e = 0; e < 4 && n + e < g.N; ++e) crow[n + e] = v[e];
        }
      }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int RS, bool KTAIL, bool SILU, bool BNM = false>
int launch_mfma(const MfmaArgs& g, hipStream_t s) {
  const int64_t tiles = int64_t((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  if (tiles > INT32_MAX) return invalid("matmul: matrix too large");
  hipLaunchKernelGGL((gemm_mfma_nt<BM, BN, WAVES_M, WAVES_N, RS, KTAIL, SILU, false, BNM>), dim3(unsigned(tiles)),
                     dim3(WAVES_M * WAVES_N * 64), 0, s, g);
  return check_launch("matmul");
}

// Tile shape by a cost model fitted on MI355X at the Qwen3-0.6B projections: a launch runs in ceil(tiles / 256)
// rounds of one tile per CU, so its time goes as rounds x tile area / efficiency, the efficiency of a tile growing
// with its size (fewer L2 bytes per flop). At M = 2048 this picks 128x256 for N = 4096, 256x192 for N = 6144 and
// 64x128 for N = 1024 -- 256 tiles each, the fastest of a sweep over eleven shapes.
// When 64x64 tiles fit in one round (M <= 64, or mixed steps and prefill chunks of up to a few hundred rows) a
// block's time is its chain of K / 64 k-tiles, each waiting on its loads: 64x64 tiles with 4 k-tiles of loads in
// flight (RS = 4) instead of 2 (M = 256: down 22.6 -> 15.8 us, o_proj 15.4 -> 11.0, qkv 9.9 -> 7.4; deeper
// staging measured no faster, and none of it helps once every CU has a large tile), and 32x64 tiles where those
// still fit one round (more blocks, each streaming fewer bytes). The k order of every tile
// shape is the same, so the result does not depend on the choice.
template <int RS, bool KTAIL, bool SILU, bool BNM = false>
int launch_mfma_shape(const MfmaArgs& g, hipStream_t s) {
  constexpr int kCUs = 256;
  const int64_t tiles64 = int64_t((g.M + 63) / 64) * ((g.N + 63) / 64);
  if (g.M <= 64 || tiles64 <= kCUs) {
    // 32 x 64 tiles (2 waves) when they still fit one round: twice the blocks of 64 x 64 (K = 1024, weights from
    // HBM: qkv M = 48 / 64 / 96 / 128 7.2 / 7.7 / 7.2 / 7.5 -> 6.4 / 6.6 / 6.5 / 6.5 us, gate_up M = 48 / 64 7.5 /
    // 7.9 -> 6.5 / 6.8 us); past one round (or with 8 k-tiles in flight) they measured slower
    const int64_t tiles32 = int64_t((g.M + 31) / 32) * ((g.N + 63) / 64);
    if constexpr (!KTAIL)
      if (g.M > 32 && tiles32 <= kCUs && ((g.K / kBK) & 3) == 0)
        return launch_mfma<32, 64, 1, 2, 4, false, SILU, BNM>(g, s);
    if constexpr (!KTAIL)
      if (((g.K / kBK) & 3) == 0) return launch_mfma<64, 64, 2, 2, 4, false, SILU, BNM>(g, s);
    return launch_mfma<64, 64, 2, 2, RS, KTAIL, SILU, BNM>(g, s);
  }
  struct Shape { int bm, bn; double eff; };
  constexpr Shape shapes[] = {{256, 256, 1.0}, {256, 192, 1.0}, {128, 256, 0.95}, {128, 128, 0.85}, {64, 128, 0.75}};
  int best = 0;
  double best_cost = 0.0;
  for (int i = 0; i < 5; ++i) {
    const int64_t tiles = int64_t((g.M + shapes[i].bm - 1) / shapes[i].bm) * ((g.N + shapes[i].bn - 1) / shapes[i].bn);
    const double cost = double((tiles + kCUs - 1) / kCUs) * shapes[i].bm * shapes[i].bn / shapes[i].eff;
    if (i == 0 || cost < best_cost) best = i, best_cost = cost;
  }
  switch (best) {
    case 0: return launch_mfma<256, 256, 4, 2, 1, KTAIL, SILU, BNM>(g, s);
    case 1: return launch_mfma<256, 192, 4, 2, RS, KTAIL, SILU, BNM>(g, s);
    case 2: return launch_mfma<128, 256, 2, 4, RS, KTAIL, SILU, BNM>(g, s);  // 8 waves of 64x64: 3 % faster than 4 of 64x128
    case 3: return launch_mfma<128, 128, 2, 4, RS, KTAIL, SILU, BNM>(g, s);
    default: return launch_mfma<64, 128, 2, 2, RS, KTAIL, SILU, BNM>(g, s);
  }
}

// N-contiguous B: the tile kernel at every M (the skinny kernels read K-contiguous W rows straight into MFMA
// operands).
int launch_mfma_bnm(const MfmaArgs& g, hipStream_t s) {
  const int nk = (g.K + kBK - 1) / kBK;
  if (g.K % kBK != 0) return launch_mfma_shape<1, true, false, true>(g, s);
  if (nk % 2 == 0) return launch_mfma_shape<2, false, false, true>(g, s);
  return launch_mfma_shape<1, false, false, true>(g, s);
}

// 8 waves per block; 4 k steps of loads per wave in flight for wide outputs and 8-column blocks, 8 for 16-column
// blocks when N < 2048 -- the best of sweeps over 4/8/12/16 waves and 2/4/8/12 steps at the Qwen3-0.6B shapes.
// Block tile: all rows (MT = ceil(M / 16) row tiles) x 16 columns when that gives >= 256 blocks; else one 16-row
// tile per block (grid.y = row tiles) x 16 columns, or x 8 columns. One CU streams at most ~70 GB/s from L2/HBM,
// and every block reads all of its rows of A (32 x K: twice the W slice of a 16-column block), so narrow outputs
// (N = 1024: 64 blocks of 32 x 16) need the smaller tiles to reach every CU.
// 8-column blocks with K >= 2048 (o_proj, down_proj) stage their operands through LDS (gemm_skinny_lds, same bits):
// o_proj 5.75 -> 4.58 us, down 7.81 -> 6.04 us with the weights from HBM. 16-column blocks with 512 < K <= 1024
// (qkv, gate_up) stage the whole K in one round (every load of the block in flight at once, 16-byte loads along
// the rows instead of fragments of half a 128-byte line per row): M = 32 qkv 5.38 -> 4.74 us, the 6144-wide gate_up
// product 8.17 -> 7.61 us, M = 16 4.45 -> 4.25 / 6.28 -> 5.33 us (staged in rounds of 256 k they had measured
// within 4 % or slower: a barrier and an LDS round trip per round).
template <int MT, int NCOL, bool SILU>
int launch_skinny_tile(const MfmaArgs& g, hipStream_t s) {
  constexpr int NW = 8;
  const int nout = SILU ? g.N / 2 : g.N;
  const dim3 grid(unsigned((nout + NCOL - 1) / NCOL), unsigned((g.M + 16 * MT - 1) / (16 * MT))), block(NW * 64);
  bool done = false;
  if constexpr (NCOL == 16) {
    if (g.K > 512 && g.K <= 1024) {  // the whole K in one round of up to 1024 (staged chunks past K are zero)
      done = true;
      hipLaunchKernelGGL((gemm_skinny_lds<MT, 16, NW, 4, SILU, true>), grid, block, 0, s, g);
    }
  }
  if constexpr (NCOL == 8 && MT == 1 && !SILU) {
    if (g.K >= 2048 && g.K <= 13 * 256) {  // the whole K in one round (24 staged rows: LDS <= 160 KB)
      done = true;
      switch ((g.K + 255) / 256) {
#define NVHIP_ONE_ROUND(U) \
  case U: hipLaunchKernelGGL((gemm_skinny_lds<1, 8, NW, U, false, true>), grid, block, 0, s, g); break;
        NVHIP_ONE_ROUND(8) NVHIP_ONE_ROUND(9) NVHIP_ONE_ROUND(10) NVHIP_ONE_ROUND(11) NVHIP_ONE_ROUND(12)
        default: hipLaunchKernelGGL((gemm_skinny_lds<1, 8, NW, 13, false, true>), grid, block, 0, s, g);
#undef NVHIP_ONE_ROUND
      }
    }
  }
  if (done) {
  } else if (NCOL == 8 && MT == 1 && g.K >= 2048) hipLaunchKernelGGL((gemm_skinny_lds<1, 8, NW, 4, SILU>), grid, block, 0, s, g);
  else if (g.N >= 2048 || NCOL == 8) hipLaunchKernelGGL((gemm_skinny<MT, NCOL, NW, 4, SILU>), grid, block, 0, s, g);
  else hipLaunchKernelGGL((gemm_skinny<MT, NCOL, NW, 8, SILU>), grid, block, 0, s, g);
  return check_launch("matmul");
}

template <int MT, bool SILU>
int launch_skinny(const MfmaArgs& g, hipStream_t s) {
  constexpr int64_t kBlocks = 256;
  const int64_t nout = SILU ? g.N / 2 : g.N;
  // very wide outputs (the LM head): 64 columns per block, so each block's A reads serve four times the W bytes;
  // 4 waves (a sweep of 2 / 4 / 8 / 16 waves x 2 / 4 / 8 / 16 steps x 16 / 32 / 64 columns picked 4 waves of 8 k
  // steps for gemm_skinny: 32 x 151936 x 1024 in 73.6 us vs 81.0 us with 8 waves of 4); staged through LDS one
  // 128-k round at a time (52 KB of LDS, three blocks per CU): 64.3 us (two k steps per wave and round: 86.7 us);
  // with K = 1024 (the Qwen3-0.6B LM head) gemm_wide_k1024: A staged once per block, each wave streaming W tiles
  // of 16 columns through its own LDS slice, 256 blocks of 8 waves
  if constexpr (!SILU)
    if ((nout + 63) / 64 >= 8 * kBlocks) {
      if (g.K == 1024) {
        hipLaunchKernelGGL((gemm_wide_k1024<MT>), dim3(256), dim3(512), 0, s, g);
      } else {
        const dim3 grid(unsigned((nout + 63) / 64), unsigned((g.M + 16 * MT - 1) / (16 * MT)));
        hipLaunchKernelGGL((gemm_skinny_lds<MT, 64, 4, 1, SILU>), grid, dim3(4 * 64), 0, s, g);
      }
      return check_launch("matmul");
    }
  if ((nout + 15) / 16 >= kBlocks) return launch_skinny_tile<MT, 16, SILU>(g, s);
  if (MT > 1 && MT * ((nout + 15) / 16) >= kBlocks) return launch_skinny_tile<1, 16, SILU>(g, s);
  return launch_skinny_tile<1, 8, SILU>(g, s);
}

template <int MT, int NCOL, bool SILU, int KC, bool ADD>
int launch_skinny_norm_tile(const NormMfmaArgs& a, hipStream_t s) {
  const int nout = SILU ? a.g.N / 2 : a.g.N;
  const dim3 grid(unsigned((nout + NCOL - 1) / NCOL), unsigned((a.g.M + 16 * MT - 1) / (16 * MT))), block(512);
  hipLaunchKernelGGL((gemm_skinny_norm<MT, NCOL, SILU, KC, ADD>), grid, block, 0, s, a);
  return check_launch("rms_norm_matmul");
}

// The block tiles of launch_skinny (without the 64-column one); K = 2048 keeps one 16-row tile per block so that
// the normalised rows (16 x 2056 bf16) and the reduction buffer fit the LDS.
template <bool SILU, int KC, bool ADD>
int launch_skinny_norm(const NormMfmaArgs& a, hipStream_t s) {
  const int64_t nout = SILU ? a.g.N / 2 : a.g.N, cols16 = (nout + 15) / 16;
  // all rows per block down to 192 column tiles: gate_up + SiLU (3072 outputs) on 192 blocks of 32 rows rather than
  // 384 of 16, which put two blocks on half of the CUs (decode step 1.99 -> 1.97 ms)
  // qkv (4096 outputs, K = 1024): 32 columns x 16 rows per block (256 blocks), each block's x / residual rows half
  // of the 32-row tile's: 7.14 -> 6.68 us (sweep of 16 / 32 rows x 8 / 16 / 32 columns; for gate_up + SiLU the
  // 32 x 16 tile below stays the best)
  if constexpr (KC == 4 && !SILU)
    if (a.g.M > 16 && (nout + 31) / 32 * 2 >= 256) return launch_skinny_norm_tile<1, 32, SILU, KC, ADD>(a, s);
  if constexpr (KC == 4)
    if (a.g.M > 16 && cols16 >= 192) return launch_skinny_norm_tile<2, 16, SILU, KC, ADD>(a, s);
  if (cols16 * ((a.g.M + 15) / 16) >= 256) return launch_skinny_norm_tile<1, 16, SILU, KC, ADD>(a, s);
  return launch_skinny_norm_tile<1, 8, SILU, KC, ADD>(a, s);
}

template <bool SILU>
int launch_mfma_auto(const MfmaArgs& g, hipStream_t s) {
  if (g.M <= 16) return launch_skinny<1, SILU>(g, s);
  if (g.M <= 32) return launch_skinny<2, SILU>(g, s);
  // 33 .. 256 rows with a long K (o_proj, down_proj): a block streams ~45-50 GB/s from L2 / HBM whatever the
  // kernel, so the time is the bytes of the busiest block, and 16 - 64 64x64 tiles, each a chain of K / 64 k-tiles
  // on one CU, leave most CUs idle. There the skinny kernel runs 32-row blocks as grid rows, 16 columns wide while
  // that grid fits one round on the CUs, else 32, its operands staged through LDS in rounds of 768 (16 columns) or
  // 512 k (row-contiguous loads; read straight into fragments the same blocks took 11.1 vs 7.7 us at M = 128 and
  // 14.3 vs 10.0 us at M = 256 for down_proj). Graph replay, weights from HBM, N = 1024, against the 64x64 tiles:
  // M = 64 down 17.1 -> 7.8 us, o_proj 11.7 -> 6.4; M = 128 16.4 -> 7.7 / 11.3 -> 6.3; M = 256 15.9 -> 9.9 /
  // 11.2 -> 8.3 (hipBLASLt 11.9 / 10.7, 9.6 / 10.5, 10.1 / 10.7). A row's bits depend only on its tile's rows, as
  // for M <= 32: every skinny block shape sums an output in the same k order. The choice between the skinny and the
  // tile kernels depends only on M, K and the W rows (g.N, gate and up rows together with SILU), so the SiLU x Mul
  // epilogue runs the kernel family its two-step equivalent (the plain product of the same W) runs and stays
  // bitwise equal to it.
  const int64_t rows32 = (g.M + 31) / 32;
  if (g.M <= 256 && g.K >= 2048 && rows32 * ((g.N + 31) / 32) <= 256) {
    const dim3 block(512);
    if constexpr (SILU) {  // gate and up rows: 16 output columns stage 64 rows, as 32 plain columns do
      hipLaunchKernelGGL((gemm_skinny_lds<2, 16, 8, 2, true>), dim3(unsigned((g.N / 2 + 15) / 16), unsigned(rows32)),
                         block, 0, s, g);
    } else if (rows32 * ((g.N + 15) / 16) <= 256) {
      hipLaunchKernelGGL((gemm_skinny_lds<2, 16, 8, 3, false>), dim3(unsigned((g.N + 15) / 16), unsigned(rows32)),
                         block, 0, s, g);
    } else {
      hipLaunchKernelGGL((gemm_skinny_lds<2, 32, 8, 2, false>), dim3(unsigned((g.N + 31) / 32), unsigned(rows32)),
                         block, 0, s, g);
    }
    return check_launch("matmul");
  }
  if (g.M <= 64 && g.K >= 2048) return launch_skinny<2, SILU>(g, s);  // wider outputs: the M <= 32 tilings
  const int nk = (g.K + kBK - 1) / kBK;
  if (g.K % kBK != 0) return launch_mfma_shape<1, true, SILU>(g, s);
  if (nk % 2 == 0) return launch_mfma_shape<2, false, SILU>(g, s);
  return launch_mfma_shape<1, false, SILU>(g, s);
}

// 256x256 tiles (16 waves, 16-byte fragment reads) when they fill the CUs at least once, else 128x128 (8 waves).
// 4096^3 "ieee" with an N-contiguous B: 1051 us with gemm_mfma_f32<256, 256, 4, 4> -> 982 us (torch.matmul 914 us);
// 128x128 / 256x256 tiles with 4 or 8 waves of 64x64 .. 128x128 measured 1042-1108 us. The tf32 rounding adds
// registers that the next group's fragments would spill, so that variant reads them as it goes.
template <bool B_NMAJOR, bool TF32>
int launch_f32(const F32Args& g, hipStream_t s) {
  const int64_t big = int64_t((g.M + 255) / 256) * ((g.N + 255) / 256);
  if (big >= 256) {
    if (big > INT32_MAX) return invalid("matmul: matrix too large");
    hipLaunchKernelGGL((gemm_mfma_f32q<256, 256, 4, 4, B_NMAJOR, TF32, !TF32>), dim3(unsigned(big)), dim3(1024), 0, s,
                       g);
    return check_launch("matmul");
  }
  const int64_t tiles = int64_t((g.M + 127) / 128) * ((g.N + 127) / 128);
  if (tiles > INT32_MAX) return invalid("matmul: matrix too large");
  hipLaunchKernelGGL((gemm_mfma_f32<128, 128, 2, 4, B_NMAJOR, TF32>), dim3(unsigned(tiles)), dim3(512), 0, s, g);
  return check_launch("matmul");
}

template <typename T, bool TF32>
int launch_generic(const GemmArgs& g, hipStream_t s) {
  const int64_t gx = (g.N + 63) / 64, gy = (g.M + 63) / 64;
  if (gx > INT32_MAX || gy > 65535) return invalid("matmul: matrix too large");
  hipLaunchKernelGGL((gemm_generic<T, TF32>), dim3(unsigned(gx), unsigned(gy)), dim3(kBlock), 0, s, g);
  return check_launch("matmul");
}

}  // namespace
}  // namespace nvhip

extern "C" int nvhip_matmul(void* c, const void* a, const void* b, int64_t M, int64_t N, int64_t K, int64_t sam,
                            int64_t sak, int64_t sbk, int64_t sbn, int64_t scm, int64_t scn, int dtype,
                            int precision, void* stream) {
  using namespace nvhip;
  clear_error();
  if (M < 0 || N < 0 || K < 0) return invalid("matmul: negative size");
  if (sam < 0 || sak < 0 || sbk < 0 || sbn < 0 || scm < 0 || scn < 0) return invalid("matmul: negative stride");
  if (dtype != NVHIP_DTYPE_F32 && dtype != NVHIP_DTYPE_BF16) return invalid("matmul: dtype must be fp32 or bf16");
  if (precision != NVHIP_PREC_IEEE && precision != NVHIP_PREC_TF32)
    return invalid("matmul: precision must be ieee or tf32");
  if (M == 0 || N == 0) return NVHIP_OK;
  if (!c || (K > 0 && (!a || !b))) return invalid("matmul: null pointer");
  GemmArgs g{c, a, b, M, N, K, sam, sak, sbk, sbn, scm, scn};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == NVHIP_DTYPE_BF16) {
    // MFMA path: A and B K-contiguous with 16-byte aligned rows, C with unit column stride, sizes within int32
    const bool nt = sak == 1 && sbk == 1 && scn == 1 && K % 8 == 0 && K > 0 && sam % 8 == 0 && sbn % 8 == 0 &&
                    aligned16(a) && aligned16(b) &&
                    M < (int64_t(1) << 31) && N < (int64_t(1) << 31) && K < (int64_t(1) << 31);
    if (nt) {
      MfmaArgs m{static_cast<uint16_t*>(c), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                 int(M), int(N), int(K), sam, sbn, scm};
      return launch_mfma_auto<false>(m, s);
    }
    // MFMA path for an N-contiguous B ([K, N] row-major): 16-byte aligned rows of A (K-contiguous) and B, N % 8 == 0
    const bool nn = sak == 1 && sbn == 1 && scn == 1 && K % 8 == 0 && K > 0 && N % 8 == 0 && sam % 8 == 0 &&
                    sbk % 8 == 0 && aligned16(a) && aligned16(b) &&
                    M < (int64_t(1) << 31) && N < (int64_t(1) << 31) && K < (int64_t(1) << 31);
    if (nn) {
      MfmaArgs m{static_cast<uint16_t*>(c), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                 int(M), int(N), int(K), sam, sbk, scm};
      return launch_mfma_bnm(m, s);
    }
    return launch_generic<uint16_t, false>(g, s);
  }
  // fp32 MFMA path: A K-contiguous, B K- or N-contiguous, 16-byte aligned rows, C with unit column stride
  const bool tf32 = precision == NVHIP_PREC_TF32;
  const bool b_kmajor = sbk == 1 && sbn % 4 == 0, b_nmajor = sbn == 1 && sbk % 4 == 0 && N % 4 == 0;
  const bool mfma = sak == 1 && sam % 4 == 0 && K % 4 == 0 && K > 0 && scn == 1 && (b_kmajor || b_nmajor) &&
                    aligned16(a) && aligned16(b) &&
                    M < (int64_t(1) << 31) && N < (int64_t(1) << 31) && K < (int64_t(1) << 31);
  if (mfma) {
    F32Args f{static_cast<float*>(c), static_cast<const float*>(a), static_cast<const float*>(b),
              int(M), int(N), int(K), sam, sbk, sbn, scm};
    if (b_kmajor) return tf32 ? launch_f32<false, true>(f, s) : launch_f32<false, false>(f, s);
    return tf32 ? launch_f32<true, true>(f, s) : launch_f32<true, false>(f, s);
  }
  if (tf32) return launch_generic<float, true>(g, s);
  return launch_generic<float, false>(g, s);
}

extern "C" int nvhip_matmul_silu_mul_bf16(void* out, const void* a, const void* w, int64_t M, int64_t N2, int64_t K,
                                          int64_t sam, int64_t swn, int64_t som, void* stream) {
  using namespace nvhip;
  clear_error();
  if (M < 0 || N2 < 0 || K < 0) return invalid("matmul_silu_mul: negative size");
  if (M == 0 || N2 == 0) return NVHIP_OK;
  if (!out || !a || !w) return invalid("matmul_silu_mul: null pointer");
  if (K <= 0 || K % 8 != 0 || sam % 8 != 0 || swn % 8 != 0 || sam < K || swn < K || som < N2 || !aligned16(a) ||
      !aligned16(w))
    return invalid("matmul_silu_mul: needs K % 8 == 0 and 16-byte aligned, K-contiguous rows of A and W");
  if (M >= (int64_t(1) << 31) || 2 * N2 >= (int64_t(1) << 31) || K >= (int64_t(1) << 31))
    return invalid("matmul_silu_mul: size too large");
  MfmaArgs m{static_cast<uint16_t*>(out), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(w),
             int(M), int(2 * N2), int(K), sam, swn, som};
  return launch_mfma_auto<true>(m, static_cast<hipStream_t>(stream));
}

extern "C" int nvhip_rms_norm_matmul_bf16(void* out, void* residual_out, const void* x, const void* residual,
                                          const void* norm_w, float eps, const void* w, int64_t M, int64_t N,
                                          int64_t K, int64_t sx, int64_t sr, int64_t swn, int64_t som, int silu,
                                          void* stream) {
  using namespace nvhip;
  clear_error();
  if (M < 0 || N < 0) return invalid("rms_norm_matmul: negative size");
  if (M > 32) return invalid("rms_norm_matmul: at most 32 rows (decode batches)");
  if (K != 1024 && K != 2048) return invalid("rms_norm_matmul: K (the norm width) must be 1024 or 2048");
  if (M == 0 || N == 0) return NVHIP_OK;
  const bool add = residual != nullptr;
  if (!out || !x || !norm_w || !w || (add && !residual_out) || (!add && residual_out))
    return invalid("rms_norm_matmul: null pointer (residual_out is given exactly when residual is)");
  if (sx < K || swn < K || som < N || (add && sr < K) || sx % 8 || swn % 8 || (add && sr % 8))
    return invalid("rms_norm_matmul: bad strides (K-contiguous rows, row strides multiples of 8)");
  if (!aligned16(x) || !aligned16(norm_w) || !aligned16(w) || (add && (!aligned16(residual) || !aligned16(residual_out))))
    return invalid("rms_norm_matmul: x, residual, residual_out, norm_w and w must be 16-byte aligned");
  if (add) {  // residual_out is read by no block, but x and residual are read by every block: no overlap
    const auto* ro = static_cast<const char*>(residual_out);
    const auto overlaps = [&](const void* p, int64_t stride) {
      const auto* b = static_cast<const char*>(p);
      return ro < b + ((M - 1) * stride + K) * 2 && b < ro + M * K * 2;
    };
    if (overlaps(x, sx) || overlaps(residual, sr))
      return invalid("rms_norm_matmul: residual_out must not overlap x or residual");
  }
  if (N >= (int64_t(1) << 30)) return invalid("rms_norm_matmul: N too large");
  NormMfmaArgs a{};
  a.g = MfmaArgs{static_cast<uint16_t*>(out), nullptr, static_cast<const uint16_t*>(w), int(M),
                 int(silu ? 2 * N : N), int(K), 0, swn, som};
  a.x = static_cast<const uint16_t*>(x);
  a.r = static_cast<const uint16_t*>(residual);
  a.nw = static_cast<const uint16_t*>(norm_w);
  a.res_out = static_cast<uint16_t*>(residual_out);
  a.sx = sx, a.sr = sr, a.eps = eps;
  a.factor = aten_mean_factor(K, M), a.m = aten_norm_bw(K, M) / 64;  // torch's order for a norm over M rows
  hipStream_t s = static_cast<hipStream_t>(stream);
#define NVHIP_NORM_MM(SI, V, AD) return launch_skinny_norm<SI, V, AD>(a, s)
  if (K == 1024) {
    if (silu) { if (add) NVHIP_NORM_MM(true, 4, true); NVHIP_NORM_MM(true, 4, false); }
    if (add) NVHIP_NORM_MM(false, 4, true);
    NVHIP_NORM_MM(false, 4, false);
  }
  if (silu) { if (add) NVHIP_NORM_MM(true, 8, true); NVHIP_NORM_MM(true, 8, false); }
  if (add) NVHIP_NORM_MM(false, 8, true);
  NVHIP_NORM_MM(false, 8, false);
#undef NVHIP_NORM_MM
}

namespace nvhip {
namespace {

// K ranges of the product in nvhip_matmul_add_rms_norm_bf16: when its 64x64 tiles leave CUs idle (M of a mixed step
// or a prompt chunk, N = hidden), each tile's K is split in up to 4 ranges so that every CU streams a part -- the
// blocks of a few-tile launch each wait on their chain of K / 64 k-tiles -- and the Add+RMSNorm that consumes the
// product sums the fp32 partials (no extra launch). Each range is a whole number of 4-k-tile rounds (RS = 4).
int norm_splits(int64_t M, int64_t N, int64_t K) {
  if (M <= 32 || M >= (int64_t(1) << 31) || N % 64 != 0 || K % kBK != 0 || K >= (int64_t(1) << 31) ||
      !add_rms_norm_partials_supported(N))
    return 1;
  const int64_t tiles = (M + 63) / 64 * (N / 64);
  if (tiles >= 256) return 1;
  for (int s = int(std::min<int64_t>(4, 256 / tiles)); s > 1; --s)
    if (K % (int64_t(kBK) * 4 * s) == 0) return s;
  return 1;
}

int64_t matmul_norm_workspace(int64_t M, int64_t N, int64_t K) {
  const int s = norm_splits(M, N, K);
  const int64_t bytes = s > 1 ? int64_t(s) * M * N * 4 : M * N * 2;
  return (bytes + 15) / 16 * 16;
}

}  // namespace
}  // namespace nvhip

extern "C" int64_t nvhip_matmul_add_rms_norm_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return nvhip::matmul_norm_workspace(M, N, K);
}

extern "C" int nvhip_matmul_add_rms_norm_bf16(void* y, void* residual_out, const void* x, const void* weight,
                                              const void* residual, const void* norm_w, float eps, int64_t M,
                                              int64_t N, int64_t K, int64_t x_stride, int64_t w_stride,
                                              void* workspace, int64_t workspace_size, void* stream) {
  using namespace nvhip;
  clear_error();
  if (M < 0 || N <= 0 || K <= 0) return invalid("matmul_add_rms_norm: bad shape");
  if (x_stride < K || w_stride < K || x_stride % 8 != 0 || w_stride % 8 != 0 || K % 8 != 0)
    return invalid("matmul_add_rms_norm: x / weight rows must be K-contiguous, 16-byte aligned, K % 8 == 0");
  if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) || K >= (int64_t(1) << 31))
    return invalid("matmul_add_rms_norm: size too large");
  if (M == 0) return NVHIP_OK;
  if (!y || !residual_out || !x || !weight || !residual || !norm_w || !workspace)
    return invalid("matmul_add_rms_norm: null pointer");
  if (!aligned16(y) || !aligned16(residual_out) || !aligned16(x) || !aligned16(weight) || !aligned16(residual) ||
      !aligned16(norm_w) || !aligned16(workspace))
    return invalid("matmul_add_rms_norm: pointers must be 16-byte aligned");
  if (workspace_size < matmul_norm_workspace(M, N, K))
    return invalid("matmul_add_rms_norm: workspace smaller than nvhip_matmul_add_rms_norm_workspace_size");
  hipStream_t s = static_cast<hipStream_t>(stream);
  MfmaArgs m{nullptr, static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight), int(M), int(N), int(K),
             x_stride, w_stride, N};
  const int splits = norm_splits(M, N, K);
  if (splits > 1) {  // split-K partials, summed by the norm
    m.splits = splits;
    m.ws = static_cast<float*>(workspace);
    const int64_t blocks = (M + 63) / 64 * (N / 64) * splits;
    hipLaunchKernelGGL((gemm_mfma_nt<64, 64, 2, 2, 4, false, false, true>), dim3(unsigned(blocks)), dim3(256), 0, s,
                       m);
    if (int rc = check_launch("matmul_add_rms_norm")) return rc;
    return add_rms_norm_partials(static_cast<uint16_t*>(y), static_cast<uint16_t*>(residual_out), m.ws, splits,
                                 static_cast<const uint16_t*>(residual), static_cast<const uint16_t*>(norm_w), M, N,
                                 eps, s);
  }
  // the bf16 product in the workspace, then the Add+RMSNorm: bitwise matmul followed by add_rms_norm
  m.c = static_cast<uint16_t*>(workspace);
  if (int rc = launch_mfma_auto<false>(m, s)) return rc;
  return nvhip_add_rms_norm_bf16(y, residual_out, workspace, residual, norm_w, M, N, N, N, eps, stream);
}
