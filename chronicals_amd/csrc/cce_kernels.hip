// Fused linear cross-entropy (Cut Cross-Entropy) for MI355X / gfx950.
//
// The lm_head projection S = H . W^T (H [N,d] bf16, W [V,d] bf16) and the
// softmax cross-entropy over the vocabulary are computed without ever writing
// the N x V logits to HBM:
//
//   forward   one bf16 MFMA GEMM over (256-row tile) x (run of 256-column
//             vocabulary tiles) whose epilogue keeps a per-row online
//             (max, sum-exp) in registers; a per-row combine kernel merges the
//             vocabulary splits, gathers the target logit and forms the loss.
//   backward  per vocabulary band (chunk_size columns): a recompute GEMM
//             whose epilogue forms G = dLoss/dS in bf16 for the band
//             (softmax - one-hot, masking, scaling), then two MFMA GEMMs
//             dH += G . W_band and dW_band = G^T . H.  Only the band of G
//             (N x chunk) exists in memory; its size is bounded by chunk_size.
//
// Semantics follow chronicals/kernels/cut_cross_entropy.py (reference):
//   forward   :567-692  lse = m + log(s + 1e-10); ce = lse - t;
//                        (1-eps)*ce + eps*log(V); + z*lse^2; masked mean
//   backward  :703-808  G = P - (1-eps)*onehot - eps/V + 2z*lse*P,
//                        times valid * grad_out / n_valid; dH = G W; dW = G^T H
// with the one-hot term applied (the reference's CPU path drops it at
// :773-780; its GPU path :530-546 and triton_kernels.py:2594-2601 apply it).
//
// All device work is launched on the caller's stream; there are no host
// synchronisations and no device allocations: scratch memory is a caller
// workspace whose size the *_workspace_bytes entry points report.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <float.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "../../include/chronicals_cce.h"

namespace {

typedef uint16_t bf16_t;  // raw bf16 storage
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Per-GEMM configuration: wave layout W (8 or 4), column tile BN and main-loop
// pipeline PIPE (4: direct-to-LDS loads, needs K-major operands with K a
// multiple of 64; 5: as 4 with an MN-major A read back transposed; 3:
// register-staged loads, any K).  The "fallback" configuration serves
// K % 64 != 0.
constexpr int kWarp8 = 8;
constexpr int kFastBN = 256;    // PIPE 4 kernels
constexpr int kSlowBN = 128;    // PIPE 3 kernels

constexpr int kBM = 256;              // rows of a workgroup tile
constexpr int kBK = 64;               // K slab per pipeline step
constexpr int kPitch = kBK + 8;       // LDS row pitch in bf16 (144 B: conflict-free b128 reads)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kNegBig = -FLT_MAX;   // finite "minus infinity" for running maxima

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// v_mfma_f32_32x32x16_bf16 (on gfx950 it issues at about twice the rate of
// the 16x16x32 form, measured: ~2.2 vs ~0.8-1.2 PFLOP/s device-wide).
__device__ inline f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Two floats -> packed bf16 pair (round to nearest even): one
// v_cvt_pk_bf16_f32 on gfx950.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ inline float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// ---------------------------------------------------------------------------
// Workgroup -> tile mapping.  The hardware deals consecutive workgroup ids to
// the 8 XCDs round-robin; remap so that each XCD receives a contiguous range
// of logical tiles, then walk logical tiles in groups of G row tiles so the
// ~32 workgroups resident on one XCD share G row tiles of A and 32/G column
// tiles of B through that XCD's L2 (G = 4 by default; the forward, whose
// K = d is short, measured best with G = 8).
// ---------------------------------------------------------------------------
template <int G = 4>
__device__ inline void grouped_map(int bid, int nb, int gm, int gn, int& pm, int& pn) {
  const int per = nb >> 3;
  const int u = (bid < per * 8) ? ((bid & 7) * per + (bid >> 3)) : bid;
  const int width = G * gn;
  const int grp = u / width;
  const int first = grp * G;
  const int rows = min(gm - first, G);
  const int r = u - grp * width;
  pm = first + r % rows;
  pn = r / rows;
}

// ---------------------------------------------------------------------------
// Global -> LDS operand loaders.  LDS holds every operand tile as [row][k]
// (k contiguous, pitch kPitch) so one MFMA fragment read serves both layouts.
// ---------------------------------------------------------------------------

// 16 zero bytes in device memory: out-of-range lanes load from here.
__device__ __attribute__((aligned(16))) uint32_t g_zero16[4];

// 16-byte load that is issued unconditionally: out-of-range lanes read the
// zero block instead, so the value needs no select after the load.  Keeping
// the load out of divergent control flow and unconsumed until its LDS store
// lets the compiler count outstanding loads exactly instead of draining them.
__device__ inline u32x4 guarded_load(const bf16_t* __restrict__ X, long off, bool ok) {
  const u32x4* p = ok ? reinterpret_cast<const u32x4*>(X + off) : reinterpret_cast<const u32x4*>(g_zero16);
  return *p;
}

// Per-kernel wave layout.  W = 8: two waves per SIMD, 64-row wave tiles,
// accumulators in VGPRs.  W = 4: one wave per SIMD, 128-row wave tiles,
// accumulators in AGPRs.  Waves form (256 / kWaveRows) x 2 over a tile.
template <int W>
struct WaveCfg {
  static constexpr int kThreads = W * 64;
  static constexpr int kWaveRows = (W == 8) ? 64 : 128;
  static constexpr int kFM = kWaveRows / 32;  // 32-row MFMA blocks per wave tile
};

// K-major operand: element (r, k) at X[r*ld + k].
template <int BR, int W>
struct LoadKMajor {
  static constexpr int kT = W * 64;
  static constexpr int kN = BR * (kBK / 8) / kT;  // 16-byte chunks per thread
  u32x4 v[kN];
  __device__ inline void load(const bf16_t* __restrict__ X, long ld, int r0, int rlim, int k0, int K,
                              int tid) {
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int c = tid + i * kT;
      const int row = c >> 3, kc = (c & 7) * 8;
      const int gr = r0 + row, gk = k0 + kc;
      v[i] = guarded_load(X, (long)gr * ld + gk, gr < rlim && gk < K);
    }
  }
  __device__ inline void store(bf16_t* S, int tid) const {
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int c = tid + i * kT;
      const int row = c >> 3, kc = (c & 7) * 8;
      *reinterpret_cast<u32x4*>(S + row * kPitch + kc) = v[i];
    }
  }
};

// MN-major operand (256-row tiles): element (r, k) at X[k*ld + r].  Each
// thread loads 4(k) x 8(r) blocks with 16-byte loads, transposes them in
// registers and writes 8-byte [r][k] pieces to LDS.  Lanes 0..15 of a wave
// walk k, so the 8-byte LDS writes of 16 lanes cover 32 distinct banks.
template <int W>
struct LoadMNMajor256 {
  static constexpr int kB = 512 / (W * 64);  // 4x8 blocks per thread
  u32x4 v[kB][4];
  __device__ inline void load(const bf16_t* __restrict__ X, long ld, int r0, int rlim, int k0, int K,
                              int tid) {
    const int w = tid >> 6, l = tid & 63;
    const int kq = l & 15;
#pragma unroll
    for (int t = 0; t < kB; ++t) {
      const int rb = (w * kB + t) * 4 + (l >> 4);
      const int gr = r0 + rb * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gk = k0 + kq * 4 + i;
        v[t][i] = guarded_load(X, (long)gk * ld + gr, gk < K && gr < rlim);
      }
    }
  }
  __device__ inline void store(bf16_t* S, int tid) const {
    const int w = tid >> 6, l = tid & 63;
    const int kq = l & 15;
#pragma unroll
    for (int t = 0; t < kB; ++t) {
      const int rb = (w * kB + t) * 4 + (l >> 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t a0 = v[t][0][q], a1 = v[t][1][q], a2 = v[t][2][q], a3 = v[t][3][q];
        const u32x2 ev = {(a0 & 0xffffu) | (a1 << 16), (a2 & 0xffffu) | (a3 << 16)};
        const u32x2 od = {(a0 >> 16) | (a1 & 0xffff0000u), (a2 >> 16) | (a3 & 0xffff0000u)};
        *reinterpret_cast<u32x2*>(S + (rb * 8 + 2 * q) * kPitch + kq * 4) = ev;
        *reinterpret_cast<u32x2*>(S + (rb * 8 + 2 * q + 1) * kPitch + kq * 4) = od;
      }
    }
  }
};

template <bool KMAJ, int BR, int W>
struct LoaderSel {
  typedef LoadKMajor<BR, W> type;
};
template <int W>
struct LoaderSel<false, 256, W> {
  typedef LoadMNMajor256<W> type;
};

// Row compaction: when `dyn` is set, `live` points at the device-side count
// of live rows (a multiple of 256, or the row count), and the operand's rows
// start at row live_base of that order (a block of rows), so the block holds
// live - live_base of them.  kDynM: M is cut to that and the row tiles past
// it do not run; kDynK: the reduction runs over those rows only.
constexpr int kDynNone = 0, kDynM = 1, kDynK = 2;

struct GemmShape {
  const bf16_t* A;  // M x K operand
  long lda;
  const bf16_t* B;  // N x K operand
  long ldb;
  int M, N, K;
  const int* live = nullptr;
  int dyn = kDynNone;
  int live_base = 0;
  // k offset of B in elements (direct-to-LDS pipelines): B's k index kb + k.
  // A slab that runs past K reads the rest of its row (zero padding or the
  // next rows' finite values); it never runs past the row's end (ld), so never
  // past B (kmajor_fits).
  int kb = 0;
  // Row map of a K-major A (PIPE 4): GEMM row m is row arow[m] of A, which
  // has arows rows in all (arows * lda * 2 bytes below 2^31 - 16).  Null:
  // row m is row m.
  const int* arow = nullptr;
  long arows = 0;
};

// Live rows of a row block that starts at row `base` of the compacted order.
__device__ inline int live_rows(const int* live, int base) { return max(0, *live - base); }

// Accumulator tile of one wave: kWaveRows rows x (BN/2) columns as
// kFM x (BN/64) blocks of 32x32 fp32.
template <int BN, int W>
struct WaveAcc {
  static constexpr int FM = WaveCfg<W>::kFM;
  static constexpr int FN = BN / 64;
  f32x16 v[FM][FN];
  __device__ inline void zero() {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[i][j][r] = 0.f;
  }
};

// Lane <-> element map of a wave tile.  The B fragment is passed as the
// instruction's first operand, so each 32x32 block holds C^T in the hardware
// layout: lane l owns row m = i*32 + (l & 31) and, for register r = 4q + e,
// column n = j*32 + 8q + 4*(l >> 5) + e — four consecutive columns per q.
template <int W>
__device__ inline int acc_row(int wm, int i, int l) {
  return wm * WaveCfg<W>::kWaveRows + i * 32 + (l & 31);
}
template <int BN>
__device__ inline int acc_col(int wn, int j, int q, int l) {
  return wn * (BN / 2) + j * 32 + q * 8 + (l >> 5) * 4;
}

// Opaque copies of the lane id and tile coordinates: epilogue address and
// mask arithmetic then cannot be hoisted above the K loop, where it would
// stay live next to the accumulators.
__device__ inline void pin_epilogue(int& l, int& tm, int& tn) {
  asm volatile("" : "+v"(l));
  asm volatile("" : "+s"(tm), "+s"(tn));
}

// ---------------------------------------------------------------------------
// Direct global -> LDS loads (PIPE 4).  A buffer load with the `lds` modifier
// writes each lane's 16 bytes straight into LDS at M0 + 16*lane, so one wave
// instruction fills 1 KB = 8 rows x 128 B of a [row][64 k] tile.  LDS rows
// are not padded; instead the 16-byte chunk c of row r lives at physical chunk
// c ^ swz(r), which keeps the MFMA fragment reads (16 or 8 lanes per phase,
// 32 consecutive rows, one chunk) on distinct banks.  Rows past the operand's
// end fall outside the buffer descriptor's range and read as zero; the
// epilogues mask them in any case.
// ---------------------------------------------------------------------------
__device__ inline int swz(int r) { return (r ^ (r >> 3)) & 7; }

// s_waitcnt immediate for vmcnt(n) alone (expcnt and lgkmcnt at their no-wait
// maxima): vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, long bytes) {
  const long cap = 0x7ffffff0L;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)(bytes < cap ? bytes : cap),
                                           0x00020000);
}

// Issue the DMA of a K-major tile: rows [r0, r0 + BR) x k [k0, k0 + 64) into
// the swizzled LDS region S.  Rows past rlim fall outside the descriptor's
// range and read as zero.  k0 goes in the scalar offset, which a raw buffer
// does not range-check: every slab must end inside its row (k0 + 64 <= ld),
// which kmajor_fits() checks on the host for every launch.
template <int BR, int W>
__device__ inline void dma_kmajor(const bf16_t* __restrict__ X, long ld, int r0, int rlim, int k0, bf16_t* S,
                                  int w, int l) {
  constexpr int kI = BR / (8 * W);  // wave instructions per wave
  const long rows_left = (long)rlim - r0;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(X + (long)r0 * ld, rows_left > 0 ? rows_left * ld * 2 : 0);
#pragma unroll
  for (int j = 0; j < kI; ++j) {
    const int blk = w * kI + j;           // 8-row block of the tile
    const int row = blk * 8 + (l >> 3);
    const int c = (l & 7) ^ swz(row);     // logical chunk this lane fetches
    const int voff = (int)(((long)row * ld + c * 8) * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rs, (__attribute__((address_space(3))) void*)(S + blk * 512), 16, voff, k0 * 2, 0, 0);
  }
}

// The K-major A tile a workgroup streams (rows [r0, r0 + kBM) of a GEMM with
// rlim rows) read through a row map: GEMM row m is row arow[m] of A, which
// has arows rows.  The buffer descriptor spans all of A; for each DMA
// instruction j of the wave, each lane keeps the byte offset of its 16-byte
// chunk at k = 0 (the slab's k0 goes in the instruction's scalar offset),
// computed once per workgroup.  Rows past rlim get an offset past the descriptor's
// range and read as zero.
template <int W>
struct ARows {
  static constexpr int kI = kBM / (8 * W);
  const bf16_t* base;
  long bytes;
  int voff[kI];
  __device__ inline void init(const bf16_t* __restrict__ X, long ld, int r0, int rlim, const int* __restrict__ arow,
                              long arows, int w, int l) {
    const long rows_left = (long)rlim - r0;
    base = X;
    bytes = arows * ld * 2;
#pragma unroll
    for (int j = 0; j < kI; ++j) {
      const int row = (w * kI + j) * 8 + (l >> 3);
      const int c = (l & 7) ^ swz(row);
      voff[j] = row < rows_left ? (int)(((long)arow[r0 + row] * ld + c * 8) * 2) : (int)0x80000000u;
    }
  }
  // the DMA of k [k0, k0 + 64) into the swizzled LDS region S
  __device__ inline void dma(int k0, bf16_t* S, int w) const {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, bytes);
#pragma unroll
    for (int j = 0; j < kI; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(S + (w * kI + j) * 512), 16, voff[j], k0 * 2, 0, 0);
  }
};

// MN-major tile for PIPE 5: element (m, k) at X[k*ld + m].  The tile
// k [k0, k0 + 64) x m [m0, m0 + 256) is copied in its natural [k][m] layout
// (512 B per k row; one wave instruction = 2 rows), with 16-byte chunk c of
// row k stored at physical chunk c ^ (4*(k & 3)) so the four rows touched by
// one transposed fragment read land on distinct banks.  Rows k >= K fall
// outside the descriptor's range and read as zero.
template <int W>
__device__ inline void dma_mnmajor256(const bf16_t* __restrict__ X, long ld, int m0, int k0, int K, bf16_t* S,
                                      int w, int l) {
  constexpr int kI = 32 / W;  // 32 wave instructions per 64 x 256 tile
  const long rows_left = (long)K - k0;
  const long bytes = rows_left > 0 ? (rows_left * ld - m0) * 2 : 0;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(X + (long)k0 * ld + m0, bytes);
#pragma unroll
  for (int j = 0; j < kI; ++j) {
    const int blk = w * kI + j;  // pair of k rows
    const int row = blk * 2 + (l >> 5);
    const int c = (l & 31) ^ (4 * (row & 3));
    const int voff = (int)(((long)row * ld + c * 8) * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rs, (__attribute__((address_space(3))) void*)(S + blk * 512), 16, voff, 0, 0, 0);
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: in each 16-lane group, lane j receives element j&3 of
// the 8-byte reads addressed by lanes (j>>2) + 4t, t = 0..3.  Lane a of the
// group addresses row k = kb + (a>>2), columns m = mb + 4*(a&3) .. +3 of the
// [k][m] tile, so lane j receives k = kb..kb+3 of column m = mb + j.
__device__ inline uint2 read_tr4(const bf16_t* S, int k, int m) {
  const int phys = (((m >> 3) ^ (4 * (k & 3))) << 3) + (m & 7);
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(S + k * 256 + phys));
  return __builtin_bit_cast(uint2, v);
}

// Register fragments of one k-step (16 of K) for a wave.
template <int BN, int W>
struct Frags {
  u32x4 a[WaveCfg<W>::kFM], b[BN / 64];
};

template <int BN, int W>
__device__ inline void read_frags(const bf16_t* __restrict__ As, const bf16_t* __restrict__ Bs, int kk,
                                  Frags<BN, W>& f, int wm, int wn, int l) {
  const int kof = kk * 16 + (l >> 5) * 8;
#pragma unroll
  for (int i = 0; i < WaveCfg<W>::kFM; ++i)
    f.a[i] = *reinterpret_cast<const u32x4*>(As + (wm * WaveCfg<W>::kWaveRows + i * 32 + (l & 31)) * kPitch + kof);
#pragma unroll
  for (int j = 0; j < BN / 64; ++j)
    f.b[j] = *reinterpret_cast<const u32x4*>(Bs + (wn * (BN / 2) + j * 32 + (l & 31)) * kPitch + kof);
}

// Fragment reads from the swizzled (unpadded, 64 bf16 per row) layout.
template <int BN, int W>
__device__ inline void read_frags_swz(const bf16_t* __restrict__ As, const bf16_t* __restrict__ Bs, int kk,
                                      Frags<BN, W>& f, int wm, int wn, int l) {
  const int c = kk * 2 + (l >> 5);
#pragma unroll
  for (int i = 0; i < WaveCfg<W>::kFM; ++i) {
    const int r = wm * WaveCfg<W>::kWaveRows + i * 32 + (l & 31);
    f.a[i] = *reinterpret_cast<const u32x4*>(As + r * 64 + ((c ^ swz(r)) << 3));
  }
#pragma unroll
  for (int j = 0; j < BN / 64; ++j) {
    const int r = wn * (BN / 2) + j * 32 + (l & 31);
    f.b[j] = *reinterpret_cast<const u32x4*>(Bs + r * 64 + ((c ^ swz(r)) << 3));
  }
}

// A fragments from the [k][m] tile with transposed reads (PIPE 5): lane l
// gets m = i*32 + (l & 31), k = kk*16 + 8*(l >> 5) + 0..7 — the same k map as
// the K-major B fragments.
template <int BN, int W>
__device__ inline void read_frags_tr(const bf16_t* __restrict__ As, const bf16_t* __restrict__ Bs, int kk,
                                     Frags<BN, W>& f, int wm, int wn, int l) {
  const int a = l & 15;
  const int kb = kk * 16 + 8 * (l >> 5) + (a >> 2);
#pragma unroll
  for (int i = 0; i < WaveCfg<W>::kFM; ++i) {
    const int mb = wm * WaveCfg<W>::kWaveRows + i * 32 + 16 * ((l >> 4) & 1) + 4 * (a & 3);
    const uint2 lo = read_tr4(As, kb, mb);
    const uint2 hi = read_tr4(As, kb + 4, mb);
    f.a[i] = u32x4{lo.x, lo.y, hi.x, hi.y};
  }
  const int c = kk * 2 + (l >> 5);
#pragma unroll
  for (int j = 0; j < BN / 64; ++j) {
    const int r = wn * (BN / 2) + j * 32 + (l & 31);
    f.b[j] = *reinterpret_cast<const u32x4*>(Bs + r * 64 + ((c ^ swz(r)) << 3));
  }
}

// v_mfma_f32_32x32x16_bf16 over the kFM x (BN/64) blocks of one k-step.
template <int BN, int W>
__device__ inline void mfma_frags(const Frags<BN, W>& f, WaveAcc<BN, W>& acc) {
#pragma unroll
  for (int i = 0; i < WaveCfg<W>::kFM; ++i)
#pragma unroll
    for (int j = 0; j < BN / 64; ++j) acc.v[i][j] = mfma_32x32x16(f.b[j], f.a[i], acc.v[i][j]);
}

// ---------------------------------------------------------------------------
// Epilogues
// ---------------------------------------------------------------------------

struct LseParams {
  const float* bias;  // [V] or null
  float* pm;          // [splits][ldp] running max (log2 units)
  float* ps;          // [splits][ldp] sum of 2^(x - max)
  long ldp;           // row stride of pm / ps
  int splits;
  int tiles_n;
};

// Vocabulary splits per row tile of a forward whose rows were compacted: the
// split count follows the device-side count of live row tiles, and
// compact_rows_kernel stores it in live[1] (split_cost picks it).
//
// Cost of s splits over gl row tiles of tn vocabulary tiles on ncu CUs, in
// tile-times: the gl*s equal workgroups run in ceil(gl*s / ncu) rounds of
// ceil(tn / s) tiles each, plus about 0.15 tile of pipeline start per
// workgroup.  The last round's idle CUs are what a good s avoids.
__host__ __device__ inline float split_cost(int gl, int tn, int s, int ncu) {
  const int rounds = (gl * s + ncu - 1) / ncu;
  return (float)rounds * ((float)((tn + s - 1) / s) + 0.15f);
}

// Forward: per-row online (max, sum-exp) in base 2 over the workgroup's run of
// vocabulary tiles; at the end one partial per (row, split) is written.
template <int BN, int W, bool HB>
struct EpiLseT {
  typedef LseParams Params;
  static constexpr bool kMultiTile = true;
  static constexpr bool kDynSplits = true;
  static constexpr int FM = WaveCfg<W>::kFM;
  struct State {
    float m[FM], s[FM];
  };
  static __device__ inline void assign(const GemmShape& g, const Params& p, int bid, int nb, int& tm,
                                       int& t0, int& t1, int& split) {
    const int gm = (g.M + kBM - 1) / kBM;
    const int S = g.dyn == kDynM ? g.live[1] : p.splits;
    if (bid >= gm * S) {  // a compacted forward uses gm * S of the nb workgroups
      t0 = t1 = 0;
      return;
    }
    int s;
    grouped_map<8>(bid, gm * S, gm, S, tm, s);
    split = s;
    t0 = (int)(((long)p.tiles_n * s) / S);
    t1 = (int)(((long)p.tiles_n * (s + 1)) / S);
  }
  static constexpr int kStores = 0;  // global stores a tile epilogue issues per wave
  static __device__ inline void init(const Params&, State& st, const GemmShape&, int, int, int) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      st.m[i] = kNegBig;
      st.s[i] = 0.f;
    }
  }
  static constexpr int kScratch = 0;  // LDS elements the epilogue stages through
  static __device__ inline void tile(const Params& p, State& st, WaveAcc<BN, W>& acc, const GemmShape& g, int tm,
                                     int tn, int wm, int wn, int l, bf16_t*) {
    constexpr int FN = BN / 64;
    pin_epilogue(l, tm, tn);
    const int c0 = tn * BN;
    if (!HB && c0 + BN <= g.N) {
      // interior tile: max over raw logits (log2e > 0 commutes with max), then
      // one fused exp2(x*log2e - m) per element
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        float mx = kNegBig;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc.v[i][j][r]);
        const float mn = fmaxf(st.m[i], mx * kLog2e);
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) sum += fast_exp2(__builtin_fmaf(acc.v[i][j][r], kLog2e, -mn));
        st.s[i] = st.s[i] * fast_exp2(st.m[i] - mn) + sum;
        st.m[i] = mn;
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
    // edge tile or bias: per-column offset, columns past V excluded
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      float mx = kNegBig;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int col = c0 + acc_col<BN>(wn, j, q, l) + e;
            if (col < g.N) mx = fmaxf(mx, (acc.v[i][j][4 * q + e] + (HB ? p.bias[col] : 0.f)) * kLog2e);
          }
      const float mn = fmaxf(st.m[i], mx);
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int col = c0 + acc_col<BN>(wn, j, q, l) + e;
            if (col < g.N) sum += fast_exp2((acc.v[i][j][4 * q + e] + (HB ? p.bias[col] : 0.f)) * kLog2e - mn);
          }
      st.s[i] = st.s[i] * fast_exp2(st.m[i] - mn) + sum;
      st.m[i] = mn;
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  static __device__ inline void merge(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
    m = mn;
  }
  static __device__ inline void finish(const Params& p, State& st, const GemmShape& g, int tm, int split,
                                       bf16_t* smem, int wm, int wn, int l) {
    // lanes l and l+32 hold the same rows
#pragma unroll
    for (int i = 0; i < FM; ++i) merge(st.m[i], st.s[i], __shfl_xor(st.m[i], 32), __shfl_xor(st.s[i], 32));
    float* red = reinterpret_cast<float*>(smem);
    if (wn == 1 && l < 32) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = acc_row<W>(wm, i, l);
        red[row] = st.m[i];
        red[kBM + row] = st.s[i];
      }
    }
    __syncthreads();
    if (wn == 0 && l < 32) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = acc_row<W>(wm, i, l);
        merge(st.m[i], st.s[i], red[row], red[kBM + row]);
        const int grow = tm * kBM + row;
        if (grow < g.M) {
          const long ldp = g.dyn == kDynM ? (long)(g.M + kBM - 1) / kBM * kBM : p.ldp;
          p.pm[(long)split * ldp + grow] = st.m[i];
          p.ps[(long)split * ldp + grow] = st.s[i];
        }
      }
    }
  }
};

template <int BN, int W>
using EpiLse = EpiLseT<BN, W, false>;
template <int BN, int W>
using EpiLseBias = EpiLseT<BN, W, true>;

struct GradParams {
  const float* bias;     // [V] or null (full vocabulary, indexed by v0 + c)
  const float4* rowp;    // [M]
  const int* rowlab;     // [M] target column or -1
  bf16_t* G;             // [M][ldg]
  long ldg;
  int v0;                // first vocabulary row of the band
  int splits;            // column-tile runs per row tile
  int tiles_n;           // column tiles in the band
};

// Backward recompute: G[n][c] = dLoss/dS for one vocabulary band, stored bf16.
// rowp[n] = {lse*log2e, cP, cT, cU}: g = cP*2^(x*log2e - lse2) - cU - cT*[c == label].
//
// Stores go through LDS: in the MFMA layout a lane holds one row, so a direct
// store instruction would touch 32 rows with 16 bytes each.  Each wave writes
// a 32 x 64 block into its own 4 KB of LDS (8-byte pieces, XOR-swizzled by
// row so the 16 lanes of a write phase hit distinct banks), reads it back
// row-major and stores whole 128-byte row segments, 8 rows per instruction.
// A wave's LDS operations execute in order, so no barrier is needed.
template <int BN, int W, bool HB>
struct EpiGradT {
  typedef GradParams Params;
  // Each workgroup walks a run of column tiles of one row tile, so the next
  // tile's loads are in flight while this tile's epilogue runs.
  static constexpr bool kMultiTile = true;
  static constexpr bool kDynSplits = false;
  static constexpr int FM = WaveCfg<W>::kFM;
  static constexpr int kScratch = W * 2048;  // 32 x 64 bf16 per wave
  // Without bias the tile epilogue issues exactly kStores buffer stores per
  // wave and no other vector memory operation (rows past M fall outside the
  // store descriptor and are dropped, so no wave branches around a store);
  // the per-row parameters are loaded once per workgroup (its row tile is
  // fixed), since a load issued after a tile's stores would wait for all of
  // them.  With bias the epilogue loads bias values, and its stores are
  // waited for in full at the next barrier (kStores = 0).
  static constexpr int kStores = HB ? 0 : FM * (BN / 128) * 4;
  static constexpr int kRows = HB ? 1 : FM;
  struct State {
    float4 rp[kRows];
    int lab[kRows];
  };
  static __device__ inline void assign(const GemmShape& g, const Params& p, int bid, int nb, int& tm, int& t0,
                                       int& t1, int& split) {
    const int gm = (g.M + kBM - 1) / kBM;
    int s;
    grouped_map(bid, nb, gm, p.splits, tm, s);
    split = s;
    t0 = (int)(((long)p.tiles_n * s) / p.splits);
    t1 = (int)(((long)p.tiles_n * (s + 1)) / p.splits);
  }
  static __device__ inline void row_params(const Params& p, const GemmShape& g, int m, float4& rp, int& lab) {
    const int mc = m < g.M ? m : 0;
    rp = p.rowp[mc];
    lab = p.rowlab[mc] - p.v0;
  }
  static __device__ inline void init(const Params& p, State& st, const GemmShape& g, int tm, int wm, int l) {
    if constexpr (!HB) {
#pragma unroll
      for (int i = 0; i < FM; ++i) row_params(p, g, tm * kBM + acc_row<W>(wm, i, l), st.rp[i], st.lab[i]);
    }
  }
  static __device__ inline void tile(const Params& p, State& st, WaveAcc<BN, W>& acc, const GemmShape& g, int tm,
                                     int tn, int wm, int wn, int l, bf16_t* scratch) {
    constexpr int FN = BN / 64;
    static_assert(FN % 2 == 0, "64-column staging blocks");
    pin_epilogue(l, tm, tn);
    bf16_t* const ws = scratch + (wm * 2 + wn) * 2048;
    const int r = l & 31;
    // this row tile of G: rows past M are out of the descriptor's range
    const int rows = min(g.M - tm * kBM, kBM);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(p.G + (long)tm * kBM * p.ldg, (long)rows * p.ldg * 2);
    // interior tile without bias: every column is inside the band and rows
    // past M are dropped by the store descriptor, so no per-element checks
    const bool interior = !HB && (tn + 1) * BN <= g.N;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = tm * kBM + acc_row<W>(wm, i, l);
      const bool mok = m < g.M;
      float4 rp;
      int lab;
      if constexpr (HB) {
        row_params(p, g, m, rp, lab);
      } else {
        rp = st.rp[i];
        lab = st.lab[i];
      }
#pragma unroll
      for (int jp = 0; jp < FN / 2; ++jp) {
        // G without the one-hot term, packed to bf16 into the staging block;
        // the 8-byte piece hc (of 16 per 128-byte row) lives at hc ^ (row & 15)
        auto stage = [&](int jj, int q, const float (&gv)[4]) {
          const int hc = (jj * 8 + 2 * q + (l >> 5)) ^ (r & 15);
          *reinterpret_cast<u32x2*>(ws + r * 64 + hc * 4) =
              u32x2{pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3])};
        };
        if (interior) {
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              float gv[4];
#pragma unroll
              for (int e = 0; e < 4; ++e)
                gv[e] = __builtin_fmaf(rp.y, fast_exp2(__builtin_fmaf(acc.v[i][2 * jp + jj][4 * q + e], kLog2e, -rp.x)),
                                       -rp.w);
              stage(jj, q, gv);
            }
        } else {
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int cb = tn * BN + acc_col<BN>(wn, 2 * jp + jj, q, l);
              float gv[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int col = cb + e;
                float gg = 0.f;
                if (mok && col < g.N) {
                  const float b = HB ? p.bias[p.v0 + col] : 0.f;
                  gg = rp.y * fast_exp2((acc.v[i][2 * jp + jj][4 * q + e] + b) * kLog2e - rp.x) - rp.w;
                }
                gv[e] = gg;
              }
              stage(jj, q, gv);
            }
        }
        asm volatile("" ::: "memory");
        // the one-hot term: the target column of row r, if it falls in this
        // 64-column block, is corrected in place by the row's first lane
        // (labels outside the band are negative or past it and never match)
        const unsigned lc = (unsigned)(lab - (tn * BN + wn * (BN / 2) + jp * 64));
        if (l < 32 && lc < 64u) {
          bf16_t* const t = ws + r * 64 + ((((int)lc >> 2) ^ (r & 15)) << 2) + (lc & 3);
          const float v = bf16_to_f32(*t) - rp.z;
          *t = __builtin_bit_cast(bf16_t, (__bf16)v);
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int rr = t * 8 + (l >> 3), c = l & 7;
          // 16-byte chunk c = pieces 2c, 2c+1, stored at slot c ^ ((rr & 14) >> 1), halves swapped for odd rows
          u32x4 v = *reinterpret_cast<const u32x4*>(ws + rr * 64 + ((c ^ ((rr & 14) >> 1)) << 3));
          if (rr & 1) v = u32x4{v[2], v[3], v[0], v[1]};
          const int trow = wm * WaveCfg<W>::kWaveRows + i * 32 + rr;
          const int gcol = tn * BN + wn * (BN / 2) + jp * 64 + c * 8;
          __builtin_amdgcn_raw_buffer_store_b128(v, gr, (int)(((long)trow * p.ldg + gcol) * 2), 0, 0);
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);  // one 64-column block live at a time
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  static __device__ inline void finish(const Params&, State&, const GemmShape&, int, int, bf16_t*, int, int,
                                       int) {}
};

template <int BN, int W>
using EpiGrad = EpiGradT<BN, W, false>;
template <int BN, int W>
using EpiGradBias = EpiGradT<BN, W, true>;

struct AccParams {
  float* acc32;
  long ldacc;
  void* out;
  long ldo;
  int out_f32;  // 0: bf16 output, 1: fp32 output
  int mode;
  const int* rowmap = nullptr;  // out row of GEMM row m (acc32 keeps GEMM rows); null: m
};

// Plain GEMM output with optional fp32 accumulation buffer.
//   mode 0: out = C            1: acc32 = C
//   mode 2: acc32 += C          3: out = acc32 + C
//   mode 4: out += C (fp32 output only: the output is its own accumulator)
template <int BN, int W>
struct EpiAcc {
  typedef AccParams Params;
  static constexpr bool kMultiTile = false;
  static constexpr bool kDynSplits = false;
  static constexpr int FM = WaveCfg<W>::kFM;
  static constexpr int kScratch = 0;
  struct State {};
  static __device__ inline void assign(const GemmShape& g, const Params&, int bid, int nb, int& tm, int& t0,
                                       int& t1, int& split) {
    const int gm = (g.M + kBM - 1) / kBM, gn = (g.N + BN - 1) / BN;
    int tn;
    grouped_map(bid, nb, gm, gn, tm, tn);
    t0 = tn;
    t1 = tn + 1;
    split = 0;
  }
  static constexpr int kStores = 0;  // single-tile workgroups: nothing follows the epilogue
  static __device__ inline void init(const Params&, State&, const GemmShape&, int, int, int) {}
  static __device__ inline void tile(const Params& p, State&, WaveAcc<BN, W>& acc, const GemmShape& g, int tm,
                                     int tn, int wm, int wn, int l, bf16_t*) {
    constexpr int FN = BN / 64;
    constexpr int JG = FN >= 2 ? 2 : 1;  // 32 x 64 column blocks whose old values load together
    pin_epilogue(l, tm, tn);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = tm * kBM + acc_row<W>(wm, i, l);
      if (m >= g.M) continue;
#pragma unroll
      for (int j0 = 0; j0 < FN; j0 += JG) {
        // the accumulator's old values for JG column blocks, all loads issued
        // before any add or store (one memory round trip per group, not per
        // 16-byte piece)
        f32x4 old[JG][4];
        const long om = p.rowmap ? (long)p.rowmap[m] : (long)m;
        if (p.mode >= 2) {
          // modes 2, 3 read the accumulator row m; mode 4 the output row om
          const float* src = p.mode == 4 ? reinterpret_cast<const float*>(p.out) + om * p.ldo
                                         : p.acc32 + (long)m * p.ldacc;
#pragma unroll
          for (int jj = 0; jj < JG; ++jj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int n = tn * BN + acc_col<BN>(wn, j0 + jj, q, l);
              old[jj][q] = n < g.N ? *reinterpret_cast<const f32x4*>(src + n) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int jj = 0; jj < JG; ++jj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int j = j0 + jj;
          const int n = tn * BN + acc_col<BN>(wn, j, q, l);
          if (n >= g.N) continue;
          f32x4 v = {acc.v[i][j][4 * q], acc.v[i][j][4 * q + 1], acc.v[i][j][4 * q + 2], acc.v[i][j][4 * q + 3]};
          if (p.mode >= 2) v += old[jj][q];
          if (p.mode == 1 || p.mode == 2) {
            *reinterpret_cast<f32x4*>(p.acc32 + (long)m * p.ldacc + n) = v;
          } else {
            if (p.out_f32) {
              *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + om * p.ldo + n) = v;
            } else {
              const u32x2 pk = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
              *reinterpret_cast<u32x2*>(reinterpret_cast<bf16_t*>(p.out) + om * p.ldo + n) = pk;
            }
          }
        }
      }
    }
  }
  static __device__ inline void finish(const Params&, State&, const GemmShape&, int, int, bf16_t*, int, int,
                                       int) {}
};

// ---------------------------------------------------------------------------
// The GEMM kernel: C[M,N] = A[M,K] . B[N,K]^T, 256 x BN x 64 tiles.  PIPE 4 / 5
// (direct-to-LDS) are described at their loop below.  PIPE 3 has two LDS
// stages and two register sets of prefetched slabs.
//
// PIPE 3 software pipeline (per slab s, LDS stage p = s & 1):
//   - global loads of slab s+2 go to register set p (issued unconditionally:
//     past the last slab the loaders' bounds predicates read zeros, so the
//     compiler's outstanding-load counts stay exact);
//   - register set p^1 (slab s+1, loaded one slab earlier) drains into LDS
//     stage p^1 after the first k-step;
//   - the fragments of k-step kk+1 are read from LDS while the MFMAs of
//     k-step kk run, and the first fragments of slab s+1 right after the
//     barrier that closes slab s.
// Tiles are walked in an even number of slabs (the loaders zero-fill past
// K) so register-set and LDS-stage parities are static in the unrolled loop.
// A workgroup may own a run of column tiles (forward); the pipeline then runs
// on across tile boundaries.  Single-tile epilogues peel the last slab pair so
// no prefetch registers are live while they run.
// ---------------------------------------------------------------------------
// LDS elements of the pipeline stages: unpadded for the direct-to-LDS
// pipelines, kPitch-padded rows for the register-staged ones.
template <int BN>
constexpr int gemm_lds_elems(int pipe, int nst = 2) {
  return (pipe >= 4 ? nst : 2) * (kBM + BN) * (pipe >= 4 ? 64 : kPitch);
}

// AROW: A is read through g.arow (PIPE 4; see ARows).
template <int BN, int W, bool AK, bool BKM, template <int, int> class EpiT, int PIPE, int NST = 2, bool AROW = false>
__device__ __forceinline__ void gemm_body(const GemmShape& g_in, const typename EpiT<BN, W>::Params& ep, int bid,
                                          int nb, bf16_t* smem) {
  static_assert(PIPE >= 3 && PIPE <= 5, "pipelines: 3 (register-staged), 4 and 5 (direct-to-LDS)");
  typedef EpiT<BN, W> Epi;
  GemmShape g = g_in;
  if (g.dyn == kDynK) g.K = min(g.K, live_rows(g.live, g.live_base));
  if (g.dyn == kDynM) {
    // Only the row tiles below the live rows run.  Epilogues with
    // kDynSplits re-split the vocabulary over all nb workgroups themselves;
    // otherwise the live tiles are spread over the first nb * live_tiles /
    // row_tiles workgroups (nb is a multiple of the row tile count for every
    // row-dynamic launch), so that every XCD keeps an equal share, and the
    // remaining workgroups exit.
    const int gm = (g.M + kBM - 1) / kBM;
    g.M = min(g.M, live_rows(g.live, g.live_base));
    if constexpr (!Epi::kDynSplits) {
      nb = nb / gm * ((g.M + kBM - 1) / kBM);
      if (bid >= nb) return;
    }
  }
  constexpr int kStage = (kBM + BN) * kPitch;
  // epilogue staging area, past the pipeline's LDS stages
  bf16_t* const scratch = smem + gemm_lds_elems<BN>(PIPE, NST);

  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;

  int tm, t0, t1, split;
  Epi::assign(g, ep, bid, nb, tm, t0, t1, split);
  if (t0 >= t1) return;  // uniform for the whole workgroup

  typename Epi::State st;
  Epi::init(ep, st, g, tm, wm, l);
  WaveAcc<BN, W> acc;

  const int KT = (g.K + kBK - 1) / kBK;
  const int KT2 = (KT + 1) & ~1;
  const int a_r0 = tm * kBM;
  bf16_t* const S0 = smem;
  bf16_t* const S1 = smem + kStage;

  if constexpr (PIPE == 4 || PIPE == 5) {
    // Direct-to-LDS pipeline over the workgroup's slabs s = 0, 1, ... (a run
    // of column tiles times KT slabs each), LDS stage s & 1.  Per slab:
    //   k-steps 0..2: MFMAs, with the fragments of the next k-step read
    //                 from LDS behind them;
    //   barrier B_s:  its implied vmcnt(0) / lgkmcnt(0) mean slab s+1's DMA
    //                 (issued after B_{s-1}) has landed for every wave and no
    //                 wave still reads slab s's stage;
    //   then the DMA of slab s+2 into that stage and the first fragments of
    //   slab s+1 are issued while the MFMAs of k-step 3 (whose fragments are
    //   already in registers) run, so the barrier's read bubble is hidden.
    // B is K-major; A is K-major (PIPE 4) or MN-major read back transposed
    // (PIPE 5).  K-major operands need K a multiple of 64 (or zero padding).
    static_assert(BKM && (PIPE == 5 || AK), "direct-to-LDS operand layouts");
    static_assert(PIPE == 4 || (!AK && BN <= 256), "PIPE 5 reads an MN-major A");
    constexpr int kSt = (kBM + BN) * 64;  // unpadded stage
    static_assert(NST >= 2 && NST <= 3, "LDS holds two or three stages");
    // DMA wave instructions per wave per slab
    constexpr int kD = (PIPE == 4 ? kBM / (8 * W) : 32 / W) + BN / (8 * W);
    auto frags = [&](const bf16_t* Sc, int kk, Frags<BN, W>& f) {
      if constexpr (PIPE == 4)
        read_frags_swz<BN, W>(Sc, Sc + kBM * 64, kk, f, wm, wn, l);
      else
        read_frags_tr<BN, W>(Sc, Sc + kBM * 64, kk, f, wm, wn, l);
    };
    // DMA of the next unissued slab (tile it2, k-slab ik2) into stage S
    int it2 = t0, ik2 = 0;
    // A through a row map: its lane offsets are computed once per workgroup
    static_assert(!AROW || PIPE == 4, "row-mapped A is K-major");
    ARows<W> arows;
    if constexpr (AROW) arows.init(g.A, g.lda, a_r0, g.M, g.arow, g.arows, w, l);
    auto issue = [&](bf16_t* S) {
      if constexpr (AROW)
        arows.dma(ik2 * kBK, S, w);
      else if constexpr (PIPE == 4)
        dma_kmajor<kBM, W>(g.A, g.lda, a_r0, g.M, ik2 * kBK, S, w, l);
      else
        dma_mnmajor256<W>(g.A, g.lda, a_r0, ik2 * kBK, g.K, S, w, l);
      dma_kmajor<BN, W>(g.B, g.ldb, it2 * BN, g.N, g.kb + ik2 * kBK, S + kBM * 64, w, l);
      if (++ik2 == KT) {
        ik2 = 0;
        ++it2;
      }
    };
    // The DMA's LDS writes count on vmcnt; the barrier's own fence does not
    // reliably wait for them, so each barrier B_s that publishes slab s+1 is
    // preceded by an explicit wait.  Vector memory operations retire in
    // issue order, so B_s may leave in flight exactly what was issued after
    // slab s+1's DMA: the DMAs of slabs s+2 .. s+NST-1, and the previous
    // tile's epilogue stores for the first NST-1 slabs of a tile (they then
    // drain behind the MFMAs).  Near the end of the run, where some of those
    // DMAs were never issued, it waits for everything.  sched_barrier fences
    // keep the MFMAs on their side of the barrier.
    auto publish = [&](int s_, bool after_epilogue) {
      __builtin_amdgcn_sched_barrier(0);
      const bool deep = s_ + NST - 1 < ((t1 - t0) * KT);
      if (deep && Epi::kStores > 0 && after_epilogue)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * kD + Epi::kStores));
      else if (deep && NST > 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * kD));
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
    };
    // each k-step: the next k-step's fragment reads are issued first, then
    // the MFMAs they hide behind
    auto order = [&]() {
      constexpr int kReads = (PIPE == 4 ? 1 : 2) * WaveCfg<W>::kFM + BN / 64;
      __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, WaveCfg<W>::kFM * (BN / 64), 0);
    };
    const int total = (t1 - t0) * KT;
    // prologue: slabs 0 .. NST-1 in flight, wait for slab 0
    issue(smem);
    if (total > 1) issue(smem + kSt);
    if constexpr (NST == 3) {
      if (total > 2) issue(smem + 2 * kSt);
    }
    // wait for slab 0 only: after its DMA come those of slabs 1 .. NST-1
    // (all issued when total > NST)
    __builtin_amdgcn_sched_barrier(0);
    if (total > NST)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NST - 1) * kD) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    Frags<BN, W> fa, fb;
    frags(smem, 0, fa);
    int s = 0, cur = 0;  // cur = s % NST
    for (int tn = t0; tn < t1; ++tn) {
      acc.zero();
      for (int kt = 0; kt < KT; ++kt, ++s) {
        const int nxt = (cur + 1 == NST) ? 0 : cur + 1;
        bf16_t* const Sc = smem + cur * kSt;
        bf16_t* const Sn = smem + nxt * kSt;
        frags(Sc, 1, fb);
        mfma_frags<BN, W>(fa, acc);
        order();
        frags(Sc, 2, fa);
        mfma_frags<BN, W>(fb, acc);
        order();
        frags(Sc, 3, fb);
        mfma_frags<BN, W>(fa, acc);
        order();
        publish(s, kt <= NST - 2 && tn != t0);  // B_s
        // the next tile's first fragments are read after this tile's
        // epilogue, so they are not live (24 VGPRs) while it runs
        if (kt + 1 < KT) frags(Sn, 0, fa);
        mfma_frags<BN, W>(fb, acc);
        order();
        __builtin_amdgcn_sched_barrier(0);
        if (s + NST < total) issue(Sc);  // stage of slab s is free after B_s
        cur = nxt;
      }
      Epi::tile(ep, st, acc, g, tm, tn, wm, wn, l, scratch);
      if (tn + 1 < t1) frags(smem + cur * kSt, 0, fa);  // slab s+1, published at B_s
    }
    Epi::finish(ep, st, g, tm, split, smem, wm, wn, l);
    return;
  }

  typename LoaderSel<AK, kBM, W>::type la0, la1;
  typename LoaderSel<BKM, BN, W>::type lb0, lb1;
  Frags<BN, W> f0, f1;

  // One slab on LDS stage P.  LOAD: refill register set P with slab (nt, nk).
  // DRAIN: store register set P^1 into stage P^1.  SYNC: close the slab with
  // a barrier and read the first fragments of the next slab.
  auto slab = [&](auto P, auto LOAD, auto DRAIN, auto SYNC, int nt, int nk) {
    constexpr int p = decltype(P)::value;
    bf16_t* const Sc = p ? S1 : S0;
    bf16_t* const Sn = p ? S0 : S1;
    auto& la = [&]() -> auto& { if constexpr (p == 0) return la0; else return la1; }();
    auto& lb = [&]() -> auto& { if constexpr (p == 0) return lb0; else return lb1; }();
    auto& la_n = [&]() -> auto& { if constexpr (p == 0) return la1; else return la0; }();
    auto& lb_n = [&]() -> auto& { if constexpr (p == 0) return lb1; else return lb0; }();
    if constexpr (decltype(LOAD)::value) {
      la.load(g.A, g.lda, a_r0, g.M, nk * kBK, g.K, tid);
      lb.load(g.B, g.ldb, nt * BN, g.N, nk * kBK, g.K, tid);
    }
    read_frags<BN, W>(Sc, Sc + kBM * kPitch, 1, f1, wm, wn, l);
    mfma_frags<BN, W>(f0, acc);
    if constexpr (decltype(DRAIN)::value) {
      la_n.store(Sn, tid);
      lb_n.store(Sn + kBM * kPitch, tid);
    }
    read_frags<BN, W>(Sc, Sc + kBM * kPitch, 2, f0, wm, wn, l);
    mfma_frags<BN, W>(f1, acc);
    read_frags<BN, W>(Sc, Sc + kBM * kPitch, 3, f1, wm, wn, l);
    mfma_frags<BN, W>(f0, acc);
    mfma_frags<BN, W>(f1, acc);
    __builtin_amdgcn_iglp_opt(0);
    if constexpr (decltype(SYNC)::value) {
      __syncthreads();
      read_frags<BN, W>(Sn, Sn + kBM * kPitch, 0, f0, wm, wn, l);
    }
  };
  typedef std::integral_constant<int, 0> I0;
  typedef std::integral_constant<int, 1> I1;
  typedef std::true_type T;
  typedef std::false_type F;

  // prologue: slabs 0 and 1 of tile t0 in flight, slab 0 in stage 0
  la0.load(g.A, g.lda, a_r0, g.M, 0, g.K, tid);
  lb0.load(g.B, g.ldb, t0 * BN, g.N, 0, g.K, tid);
  la1.load(g.A, g.lda, a_r0, g.M, kBK, g.K, tid);
  lb1.load(g.B, g.ldb, t0 * BN, g.N, kBK, g.K, tid);
  la0.store(S0, tid);
  lb0.store(S0 + kBM * kPitch, tid);
  __syncthreads();
  read_frags<BN, W>(S0, S0 + kBM * kPitch, 0, f0, wm, wn, l);

  for (int tn = t0; tn < t1; ++tn) {
    acc.zero();
    const int kt_end = Epi::kMultiTile ? KT2 : KT2 - 2;
    for (int kt = 0; kt < kt_end; kt += 2) {
      const bool w0 = kt + 2 >= KT2, w1 = kt + 3 >= KT2;
      slab(I0{}, T{}, T{}, T{}, w0 ? tn + 1 : tn, w0 ? kt + 2 - KT2 : kt + 2);
      slab(I1{}, T{}, T{}, T{}, w1 ? tn + 1 : tn, w1 ? kt + 3 - KT2 : kt + 3);
    }
    if constexpr (!Epi::kMultiTile) {
      // last slab pair of a single-tile workgroup: nothing left to load
      slab(I0{}, F{}, T{}, T{}, 0, 0);
      slab(I1{}, F{}, F{}, F{}, 0, 0);
    }
    Epi::tile(ep, st, acc, g, tm, tn, wm, wn, l, scratch);
  }
  Epi::finish(ep, st, g, tm, split, smem, wm, wn, l);
}

template <int BN, int W, bool AK, bool BKM, template <int, int> class EpiT, int PIPE, int NST = 2, bool AROW = false>
__global__ __launch_bounds__(W * 64) void gemm_kernel(GemmShape g, typename EpiT<BN, W>::Params ep) {
  __shared__ __attribute__((aligned(16))) bf16_t smem[gemm_lds_elems<BN>(PIPE, NST) + EpiT<BN, W>::kScratch];
  gemm_body<BN, W, AK, BKM, EpiT, PIPE, NST, AROW>(g, ep, blockIdx.x, gridDim.x, smem);
}

// dW and dH GEMMs of one vocabulary band in a single launch.  The first
// nb_dw workgroups take dW tiles (K = N, the longer ones), the rest dH tiles
// (K = band width), so the two tile populations pack the CUs together where
// each alone would leave a partial last wave.
template <int W, int BN_DW, int PIPE_DW, int BN_DH, int PIPE_DH>
__global__ __launch_bounds__(W * 64) void dual_acc_kernel(GemmShape g_dw, AccParams e_dw, int nb_dw, GemmShape g_dh,
                                                          AccParams e_dh) {
  constexpr int kMaxBN = BN_DW > BN_DH ? BN_DW : BN_DH;
  __shared__ __attribute__((aligned(16))) bf16_t smem[2 * (kBM + kMaxBN) * kPitch];
  if ((int)blockIdx.x < nb_dw)
    gemm_body<BN_DW, W, false, true, EpiAcc, PIPE_DW>(g_dw, e_dw, blockIdx.x, nb_dw, smem);
  else
    gemm_body<BN_DH, W, true, true, EpiAcc, PIPE_DH>(g_dh, e_dh, blockIdx.x - nb_dw, gridDim.x - nb_dw, smem);
}

// One launch per vocabulary band b of the backward (d a multiple of 64): the
// dW and dH GEMMs of band b and the logits recompute of band b+1, which
// writes the other G buffer.  Both gradient GEMMs tile d in 256-wide column
// tiles plus one 128-wide tail tile when d % 256 <= 128 (no MFMA work spent
// on padding, and the wide tiles do the most work per CU-second).
// Workgroups are numbered longest first — dW (K = N), dH (K = band width),
// then the short recompute tiles, which fill the CUs the long tiles leave
// idle at the end of the band.  The 128-wide tail tiles fit three LDS stages
// (two slabs in flight) in the space the 256-wide tiles use for two.
// The transpose of the next band's W rows (dH's B operand) rides along as the
// last, shortest population: one 64 x 64 tile per workgroup.  With dH split
// over K on very few rows, the previous band's partials are reduced by a
// population placed just before the transposes.

// dH of one band split over the band's K (few row tiles): the ks fp32
// partials P[k] = P + k * stride ([rows][d], GEMM row order) of each live row
// are summed in fixed order and applied with the band's accumulator mode, as
// the GEMM epilogue applies an unsplit tile: 0 out = s, 1 acc = s,
// 2 acc += s, 3 out = acc + s, 4 out += s (fp32 out); out rows go through the
// row map.  The rows are a block starting at row live_base of the compacted
// order (P, acc and rowmap point at the block).  d % 64 == 0.
struct DhReduce {
  const float* P;
  long stride;
  int ks, N, d;
  const int* live;
  int live_base;
  float* acc;
  int mode;
  void* out;
  int out_f32;
  const int* rowmap;
};

// Items (row, 4 columns) first, first + step, ... of a DhReduce.
__device__ inline void dh_reduce_body(const DhReduce& r, long first, long step) {
  const int rows = r.live ? min(live_rows(r.live, r.live_base), r.N) : r.N;
  const int q = r.d >> 2;
  const long total = (long)rows * q;
  for (long i = first; i < total; i += step) {
    const int m = (int)(i / q);
    const long o = (long)m * r.d + (i % q) * 4;
    f32x4 s = *reinterpret_cast<const f32x4*>(r.P + o);
    for (int k = 1; k < r.ks; ++k) s += *reinterpret_cast<const f32x4*>(r.P + k * r.stride + o);
    if (r.mode == 1 || r.mode == 2) {
      if (r.mode == 2) s = *reinterpret_cast<const f32x4*>(r.acc + o) + s;
      *reinterpret_cast<f32x4*>(r.acc + o) = s;
      continue;
    }
    if (r.mode == 3) s = *reinterpret_cast<const f32x4*>(r.acc + o) + s;
    const long oo = (long)(r.rowmap ? r.rowmap[m] : m) * r.d + (i % q) * 4;
    if (r.mode == 4) s = *reinterpret_cast<const f32x4*>(static_cast<const float*>(r.out) + oo) + s;
    if (r.out_f32)
      *reinterpret_cast<f32x4*>(static_cast<float*>(r.out) + oo) = s;
    else
      *reinterpret_cast<u32x2*>(static_cast<bf16_t*>(r.out) + oo) = u32x2{pack_bf16x2(s[0], s[1]),
                                                                           pack_bf16x2(s[2], s[3])};
  }
}

struct TransposeParams {
  const bf16_t* in;
  long ldi;
  int R, C;
  bf16_t* out;
  long ldo;
  int Rpad;
  int tiles_r;  // 64-row tiles of in
};

struct BandLaunch {
  GemmShape dw;
  AccParams e_dw;
  GemmShape dw2;
  AccParams e_dw2;
  GemmShape dh;
  AccParams e_dh;
  GemmShape dh2;
  AccParams e_dh2;
  GemmShape gr;
  GradParams e_gr;
  TransposeParams tr;
  int nb_dw, nb_dw2, nb_dh, nb_dh2, nb_gr, nb_tr;
  // dH split over the band's K (few row tiles): with dh_split each dH tile
  // has dh_ks workgroups (possibly one, for a narrow band); split k covers K
  // columns [k*dh_kc, (k+1)*dh_kc) and writes its fp32 partial with
  // e_dh*_part (mode 1) into slice k of the partial buffer (dh_part_stride
  // floats apart), which a reduction folds into the accumulator afterwards.
  int dh_split, dh_ks, dh_kc;
  long dh_part_stride;
  AccParams e_dh_part, e_dh2_part;
  // the previous band's K-split dH partials folded into the accumulator by
  // nb_red workgroups (the partials alternate between two buffers)
  DhReduce red;
  int nb_red;
};

// One split workgroup of a K-split dH population (see BandLaunch).
template <int BN, int NST>
__device__ inline void dh_split_body(const GemmShape& g0, const AccParams& e0, int ks, int kc, long stride, int b,
                                     int nb, bf16_t* smem) {
  const int k = b % ks, k0 = k * kc;
  GemmShape g = g0;
  AccParams e = e0;
  g.A += k0;
  g.B += k0;
  g.K = min(kc, g0.K - k0);
  e.acc32 += k * stride;
  gemm_body<BN, kWarp8, true, true, EpiAcc, 4, NST>(g, e, b / ks, nb / ks, smem);
}

template <int NT>
__device__ inline void transpose_tile(const bf16_t* __restrict__ in, long ldi, int R, int C, bf16_t* __restrict__ out,
                                      long ldo, int Rpad, int r0, int c0, bf16_t (*t)[66], int tid,
                                      const int* __restrict__ rmap);

// AROW: the recompute reads H's rows through the row order.
template <bool HB, bool AROW>
__global__ __launch_bounds__(kWarp8 * 64) void band_kernel(BandLaunch p) {
  __shared__ __attribute__((aligned(16))) bf16_t smem[gemm_lds_elems<kFastBN>(4) + EpiGrad<kFastBN, kWarp8>::kScratch];
  int b = blockIdx.x;
  if (b < p.nb_dw) {
    gemm_body<kFastBN, kWarp8, false, true, EpiAcc, 5>(p.dw, p.e_dw, b, p.nb_dw, smem);
    return;
  }
  b -= p.nb_dw;
  if (b < p.nb_dw2) {
    gemm_body<kSlowBN, kWarp8, false, true, EpiAcc, 5, 3>(p.dw2, p.e_dw2, b, p.nb_dw2, smem);
    return;
  }
  b -= p.nb_dw2;
  if (b < p.nb_dh) {
    if (p.dh_split)
      dh_split_body<kFastBN, 2>(p.dh, p.e_dh_part, p.dh_ks, p.dh_kc, p.dh_part_stride, b, p.nb_dh, smem);
    else
      gemm_body<kFastBN, kWarp8, true, true, EpiAcc, 4>(p.dh, p.e_dh, b, p.nb_dh, smem);
    return;
  }
  b -= p.nb_dh;
  if (b < p.nb_dh2) {
    if (p.dh_split)
      dh_split_body<kSlowBN, 3>(p.dh2, p.e_dh2_part, p.dh_ks, p.dh_kc, p.dh_part_stride, b, p.nb_dh2, smem);
    else
      gemm_body<kSlowBN, kWarp8, true, true, EpiAcc, 4, 3>(p.dh2, p.e_dh2, b, p.nb_dh2, smem);
    return;
  }
  b -= p.nb_dh2;
  if (b < p.nb_gr) {
    if constexpr (HB)
      gemm_body<kFastBN, kWarp8, true, true, EpiGradBias, 4, 2, AROW>(p.gr, p.e_gr, b, p.nb_gr, smem);
    else
      gemm_body<kFastBN, kWarp8, true, true, EpiGrad, 4, 2, AROW>(p.gr, p.e_gr, b, p.nb_gr, smem);
    return;
  }
  b -= p.nb_gr;
  if (b < p.nb_red) {
    dh_reduce_body(p.red, b * (long)(kWarp8 * 64) + threadIdx.x, (long)p.nb_red * (kWarp8 * 64));
    return;
  }
  b -= p.nb_red;
  transpose_tile<kWarp8 * 64>(p.tr.in, p.tr.ldi, p.tr.R, p.tr.C, p.tr.out, p.tr.ldo, p.tr.Rpad, (b % p.tr.tiles_r) * 64,
                              (b / p.tr.tiles_r) * 64, reinterpret_cast<bf16_t(*)[66]>(smem), threadIdx.x, nullptr);
}

// ---------------------------------------------------------------------------
// Auxiliary kernels
// ---------------------------------------------------------------------------

__device__ inline long load_label(const void* labels, int is64, long n) {
  return is64 ? reinterpret_cast<const int64_t*>(labels)[n] : (long)reinterpret_cast<const int32_t*>(labels)[n];
}

// One wave per row: merge the vocabulary-split partials into lse, gather the
// target logit (fp32 dot product of H[n] and W[label]) and form the per-row
// loss.  Each block (4 rows) writes one partial (loss sum, valid count).
__global__ __launch_bounds__(256) void fwd_combine_kernel(
    const float* __restrict__ pm, const float* __restrict__ ps, int splits, const bf16_t* __restrict__ H,
    const bf16_t* __restrict__ W, const void* labels, int labels64, const float* __restrict__ bias, int N, int d,
    int V, long ignore_index, float eps, float zw, float logV, const float* __restrict__ wsum, int labelled_only,
    const int* __restrict__ idx, const int* __restrict__ live, int nb_fwd, int tiles_n, float* __restrict__ lse_out,
    float* __restrict__ target_out, float* __restrict__ rowloss, float* __restrict__ bsum, int* __restrict__ bcnt) {
  // wave w handles partial row i; its source row is idx[i] (identity without
  // idx).  With labelled_only, ignored rows get lse 0 and their partials,
  // which the compacted GEMM may not have written, are not read.  A
  // compacted forward (live set) split the vocabulary into live[1] parts with
  // whole live tiles as the partials' row stride.
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i = blockIdx.x * 4 + w;
  long ldp = N;
  if (live) {
    const int gl = (live[0] + kBM - 1) / kBM;
    splits = live[1];
    ldp = (long)gl * kBM;
  }
  __shared__ float s_loss[4];
  __shared__ int s_cnt[4];
  float loss = 0.f;
  int cnt = 0;
  if (i < N) {
    const int n = idx ? idx[i] : i;
    const long lab = load_label(labels, labels64, n);
    const bool valid = (lab != ignore_index);
    float lse = 0.f;
    if (valid || !labelled_only) {
      float m = kNegBig, s = 0.f;
      for (int k = l; k < splits; k += 64) {
        const float m2 = pm[(long)k * ldp + i], s2 = ps[(long)k * ldp + i];
        const float mn = fmaxf(m, m2);
        s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
        m = mn;
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        const float mn = fmaxf(m, m2);
        s = s * exp2f(m - mn) + s2 * exp2f(m2 - mn);
        m = mn;
      }
      lse = m * kLn2 + logf(s + 1e-10f);
    }
    float t = 0.f;
    if (valid && lab >= 0 && lab < V) {
      const bf16_t* h = H + (long)n * d;
      const bf16_t* wr = W + lab * (long)d;
      float dot = 0.f;
      for (int k = l * 8; k < d; k += 512) {
        const u32x4 hv = *reinterpret_cast<const u32x4*>(h + k);
        const u32x4 wv = *reinterpret_cast<const u32x4*>(wr + k);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          dot += bf16_to_f32(hv[q] & 0xffffu) * bf16_to_f32(wv[q] & 0xffffu);
          dot += bf16_to_f32(hv[q] >> 16) * bf16_to_f32(wv[q] >> 16);
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o);
      t = dot + (bias ? bias[lab] : 0.f);
    }
    // uniform-target smoothing: the row mean of the logits is H[n].(sum_v W[v]) / V
    // (+ mean bias); wsum = {sum_v W[v][0..d), sum_v bias[v]}
    float smooth = logV;
    if (valid && eps > 0.f && wsum) {
      const bf16_t* h = H + (long)n * d;
      float dot = 0.f;
      for (int k = l * 8; k < d; k += 512) {
        const u32x4 hv = *reinterpret_cast<const u32x4*>(h + k);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          dot += bf16_to_f32(hv[q] & 0xffffu) * wsum[k + 2 * q];
          dot += bf16_to_f32(hv[q] >> 16) * wsum[k + 2 * q + 1];
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o);
      smooth = lse - (dot + wsum[d]) / (float)V;
    }
    if (valid) {
      float ce = lse - t;
      if (eps > 0.f) ce = (1.f - eps) * ce + eps * smooth;
      loss = ce + zw * lse * lse;
      cnt = 1;
    }
    if (l == 0) {
      lse_out[n] = lse;
      rowloss[n] = loss;
      if (target_out) target_out[n] = t;
    }
  }
  if (l == 0) {
    s_loss[w] = loss;
    s_cnt[w] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    bsum[blockIdx.x] = (s_loss[0] + s_loss[1]) + (s_loss[2] + s_loss[3]);
    bcnt[blockIdx.x] = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
  }
}

// Single block: fixed-order reduction of the block partials (deterministic).
__global__ __launch_bounds__(1024) void fwd_finalize_kernel(const float* __restrict__ bsum,
                                                            const int* __restrict__ bcnt, int nb, int reduction,
                                                            float* __restrict__ loss_out,
                                                            int32_t* __restrict__ nvalid_out) {
  __shared__ float sl[1024];
  __shared__ int sc[1024];
  float a = 0.f;
  int c = 0;
  for (int i = threadIdx.x; i < nb; i += 1024) {
    a += bsum[i];
    c += bcnt[i];
  }
  sl[threadIdx.x] = a;
  sc[threadIdx.x] = c;
  __syncthreads();
  for (int o = 512; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) {
      sl[threadIdx.x] += sl[threadIdx.x + o];
      sc[threadIdx.x] += sc[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int nv = sc[0];
    nvalid_out[0] = nv;
    if (reduction == CCE_REDUCTION_MEAN)
      loss_out[0] = sl[0] / (float)(nv > 1 ? nv : 1);
    else if (reduction == CCE_REDUCTION_SUM)
      loss_out[0] = sl[0];
  }
}

// ---------------------------------------------------------------------------
// Cross-entropy over logits that already exist (row kernels, HBM-bound).
// One 256-thread workgroup streams one row of X [N][ld] (bf16, fp16 or fp32)
// with 16-byte loads; a row whose start is not 16-byte aligned (e.g. odd V in
// bf16) takes its head and tail elements one by one.
// ---------------------------------------------------------------------------
template <typename T>
__device__ inline float elem_to_f32(T v);
template <>
__device__ inline float elem_to_f32<float>(float v) { return v; }
template <>
__device__ inline float elem_to_f32<_Float16>(_Float16 v) { return (float)v; }
template <>
__device__ inline float elem_to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <typename T>
__device__ inline T f32_to_elem(float v);
template <>
__device__ inline float f32_to_elem<float>(float v) { return v; }
template <>
__device__ inline _Float16 f32_to_elem<_Float16>(float v) { return (_Float16)v; }
template <>
__device__ inline uint16_t f32_to_elem<uint16_t>(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

// Split of row [0, V) at address p into a scalar head, 16-byte chunks and a
// scalar tail.
template <typename T>
struct RowSplit {
  static constexpr int E = 16 / sizeof(T);
  int head, chunks, tail_start;
  __device__ RowSplit(const T* p, int V) {
    const int mis = (int)((reinterpret_cast<uintptr_t>(p) & 15u) / sizeof(T));
    head = mis ? min(E - mis, V) : 0;
    chunks = (V - head) / E;
    tail_start = head + chunks * E;
  }
};

// Calls f(c, chunk) for this thread's 16-byte chunks c = tid, tid + NT, ...
// below `chunks`, issuing four loads before the first use so that every wave
// keeps 4 KB of HBM reads in flight.  kStream: non-temporal loads (data read
// once); otherwise ordinary loads, which leave the lines in the caches for a
// second read.
template <int NT = 256, bool kStream = true>
__device__ __forceinline__ u32x4 chunk_load(const u32x4* p) {
  if constexpr (kStream)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}
template <int NT = 256, bool kStream = true, typename F>
__device__ __forceinline__ void for_each_chunk(const u32x4* __restrict__ body, int chunks, int tid, F&& f) {
  constexpr int U = 4;
  int c = tid;
  for (; c + (U - 1) * NT < chunks; c += U * NT) {
    u32x4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) raw[u] = chunk_load<NT, kStream>(body + c + u * NT);
#pragma unroll
    for (int u = 0; u < U; ++u) f(c + u * NT, raw[u]);
  }
  for (; c < chunks; c += NT) f(c, chunk_load<NT, kStream>(body + c));
}

// Workgroup-wide merge of base-2 (max, sum) pairs over NW waves; every thread
// gets the result.  red holds 2*NW floats.
template <int NW = 4>
__device__ inline void block_merge_ms(float& m, float& s, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
    const float mn = fmaxf(m, m2);
    s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
    m = mn;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[2 * w] = m;
    red[2 * w + 1] = s;
  }
  __syncthreads();
  m = red[0];
  s = red[1];
#pragma unroll
  for (int k = 1; k < NW; ++k) {
    const float m2 = red[2 * k], s2 = red[2 * k + 1];
    const float mn = fmaxf(m, m2);
    s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
    m = mn;
  }
}

// Workgroup-wide sum over NW waves (fixed order); every thread gets the result.
template <int NW = 4>
__device__ inline float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();  // red may still be read by an earlier merge
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int k = 1; k < NW; ++k) t += red[k];
  return t;
}

// Forward: lse[n] = log sum exp(x), the row loss (0 for rows labelled
// ignore_index; a label outside [0, V) has no target logit)
//   CCE_SMOOTH_LOGV:    (1-eps)*(lse - x[label]) + eps*log(V)       + z*lse^2
//   CCE_SMOOTH_UNIFORM: (1-eps)*(lse - x[label]) + eps*(lse - sum(x)/V) + z*lse^2
// and one (sum, count) partial per row for fwd_finalize_kernel.
template <typename T>
__global__ __launch_bounds__(256) void ce_logits_fwd_kernel(const T* __restrict__ X, long ld, const void* labels,
                                                            int labels64, int V, long ignore_index, float eps,
                                                            float zw, float logV, int smooth_mode,
                                                            float* __restrict__ lse_out,
                                                            float* __restrict__ rowloss, float* __restrict__ bsum,
                                                            int* __restrict__ bcnt) {
  __shared__ float red[8];
  const int n = blockIdx.x, tid = threadIdx.x;
  const T* row = X + (long)n * ld;
  const RowSplit<T> sp(row, V);
  // the target logit is fetched first, so its latency hides under the stream
  long lab = 0;
  float t = 0.f;
  if (tid == 0) {
    lab = load_label(labels, labels64, n);
    if (lab != ignore_index && lab >= 0 && lab < V) t = elem_to_f32(row[lab]);
  }
  float m = kNegBig, s = 0.f;  // base 2
  float sx = 0.f;              // sum of x (natural units)
  auto add1 = [&](float x) {
    const float x2 = x * kLog2e, mn = fmaxf(m, x2);
    s = s * fast_exp2(m - mn) + fast_exp2(x2 - mn);
    m = mn;
    sx += x;
  };
  if (tid < sp.head) add1(elem_to_f32(row[tid]));
  if (tid < V - sp.tail_start) add1(elem_to_f32(row[sp.tail_start + tid]));
  const u32x4* body = reinterpret_cast<const u32x4*>(row + sp.head);
  for_each_chunk(body, sp.chunks, tid, [&](int, const u32x4& raw) {
    const T* v = reinterpret_cast<const T*>(&raw);
    float x[RowSplit<T>::E], mx = kNegBig, cs = 0.f;
#pragma unroll
    for (int e = 0; e < RowSplit<T>::E; ++e) {
      const float xe = elem_to_f32(v[e]);
      cs += xe;
      x[e] = xe * kLog2e;
      mx = fmaxf(mx, x[e]);
    }
    const float mn = fmaxf(m, mx);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < RowSplit<T>::E; ++e) acc += fast_exp2(x[e] - mn);
    s = s * fast_exp2(m - mn) + acc;
    m = mn;
    sx += cs;
  });
  block_merge_ms(m, s, red);
  if (smooth_mode == CCE_SMOOTH_UNIFORM) sx = block_sum(sx, red);
  if (tid == 0) {
    const float lse = m * kLn2 + logf(s + 1e-10f);
    const bool valid = lab != ignore_index;
    const float smooth = smooth_mode == CCE_SMOOTH_UNIFORM ? lse - sx / (float)V : logV;
    const float loss = valid ? (1.f - eps) * (lse - t) + eps * smooth + zw * lse * lse : 0.f;
    lse_out[n] = lse;
    rowloss[n] = loss;
    bsum[n] = loss;
    bcnt[n] = valid ? 1 : 0;
  }
}

// Backward: the derivative of the forward's row loss, times g_n, for valid
// rows (0 for ignored rows), with p_v = exp(x_v - lse):
//   CCE_SMOOTH_LOGV:    g_n * (((1-eps) + 2z*lse) * p_v - (1-eps) * [v == label])
//   CCE_SMOOTH_UNIFORM: g_n * ((1 + 2z*lse) * p_v - eps/V - (1-eps) * [v == label])
// g_n = grad_out[n] ('none'), grad_out[0] ('sum') or grad_out[0] / max(n_valid, 1)
// ('mean').  dX may be X itself (same dtype and stride): every element is read
// and then written by the same thread.
template <typename T, typename TO>
__global__ __launch_bounds__(256) void ce_logits_bwd_kernel(const float* __restrict__ grad_out, const T* X, long ld,
                                                            const void* labels, int labels64,
                                                            const float* __restrict__ lse,
                                                            const int32_t* __restrict__ n_valid, int V,
                                                            long ignore_index, float eps, float zw, int smooth_mode,
                                                            int reduction, TO* dX, long ldg) {
  const int n = blockIdx.x, tid = threadIdx.x;
  const T* row = X + (long)n * ld;
  TO* drow = dX + (long)n * ldg;
  const long lab = load_label(labels, labels64, n);
  const bool valid = lab != ignore_index;
  float g = reduction == CCE_REDUCTION_NONE ? grad_out[n] : grad_out[0];
  if (reduction == CCE_REDUCTION_MEAN) g /= (float)(n_valid[0] > 1 ? n_valid[0] : 1);
  const float l = lse[n];
  const bool uni = smooth_mode == CCE_SMOOTH_UNIFORM;
  const float cP = valid ? g * ((uni ? 1.f : 1.f - eps) + 2.f * zw * l) : 0.f;
  const float cU = valid && uni ? g * eps / (float)V : 0.f;
  const float cT = valid ? g * (1.f - eps) : 0.f;
  const float l2 = l * kLog2e;
  const long t = (valid && lab >= 0 && lab < V) ? lab : -1;
  auto grad1 = [&](int v, float x) { return (cP * fast_exp2(x * kLog2e - l2) - cU) - (v == t ? cT : 0.f); };
  const RowSplit<T> sp(row, V);
  // 16-byte chunks of X map onto (sizeof(TO)/sizeof(T)) aligned 16-byte
  // chunks of dX when dX's row is aligned like X's (the usual case);
  // otherwise every element goes one by one
  constexpr int E = RowSplit<T>::E;
  constexpr int kOut = sizeof(TO) / sizeof(T);
  static_assert(kOut * sizeof(T) == sizeof(TO), "output element size must be a multiple of the input's");
  const bool vec = ((reinterpret_cast<uintptr_t>(drow + sp.head) & 15u) == 0);
  if (!vec) {
    for (int v = tid; v < V; v += 256) drow[v] = f32_to_elem<TO>(grad1(v, elem_to_f32(row[v])));
    return;
  }
  if (tid < sp.head) drow[tid] = f32_to_elem<TO>(grad1(tid, elem_to_f32(row[tid])));
  if (tid < V - sp.tail_start) {
    const int v = sp.tail_start + tid;
    drow[v] = f32_to_elem<TO>(grad1(v, elem_to_f32(row[v])));
  }
  const u32x4* body = reinterpret_cast<const u32x4*>(row + sp.head);
  u32x4* dbody = reinterpret_cast<u32x4*>(drow + sp.head);
  for_each_chunk(body, sp.chunks, tid, [&](int c, const u32x4& raw) {
    const T* v = reinterpret_cast<const T*>(&raw);
    u32x4 out[kOut];
    TO* o = reinterpret_cast<TO*>(out);
    const int v0 = sp.head + c * E;
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = f32_to_elem<TO>(grad1(v0 + e, elem_to_f32(v[e])));
#pragma unroll
    for (int k = 0; k < kOut; ++k) __builtin_nontemporal_store(out[k], dbody + c * kOut + k);
  });
}

// Number of rows whose label is not ignore_index (one workgroup, fixed order).
__global__ __launch_bounds__(1024) void count_valid_kernel(const void* labels, int labels64, int N, long ignore_index,
                                                           int32_t* __restrict__ out) {
  __shared__ int part[1024];
  int c = 0;
  for (int n = threadIdx.x; n < N; n += 1024) c += load_label(labels, labels64, n) != ignore_index;
  part[threadIdx.x] = c;
  __syncthreads();
  for (int o = 512; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = part[0];
}

// Loss and gradient in one kernel: a workgroup of kFusedThreads takes rows
// n = blockIdx.x, blockIdx.x + gridDim.x, ...; for each it streams the row
// once for lse (as ce_logits_fwd_kernel) and again for the gradient (as
// ce_logits_bwd_kernel with grad_out = 1).  The grid bounds the rows in
// flight, so the second read of a row finds it in the memory-side cache.
// g_n = 1/max(n_valid,1) when n_valid is given, else 1.  dX may be X itself:
// each row's first pass ends at a barrier before its second pass writes.
constexpr int kFusedThreads = 512;
constexpr bool kFusedPass2Stream = true;  // the row's last read: non-temporal
template <typename T, typename TO>
__global__ __launch_bounds__(kFusedThreads) void ce_logits_fused_kernel(
    const T* X, long ld, const void* labels, int labels64, int N, int V, long ignore_index, float eps, float zw,
    float logV, int smooth_mode, const int32_t* __restrict__ n_valid, float* __restrict__ lse_out,
    float* __restrict__ rowloss, float* __restrict__ bsum, int* __restrict__ bcnt, TO* dX, long ldg) {
  constexpr int NW = kFusedThreads / 64;
  constexpr int E = RowSplit<T>::E;
  constexpr int kOut = sizeof(TO) / sizeof(T);
  static_assert(kOut * sizeof(T) == sizeof(TO), "output element size must be a multiple of the input's");
  __shared__ float red[2 * NW];
  const int tid = threadIdx.x;
  const float g = n_valid ? 1.f / (float)(n_valid[0] > 1 ? n_valid[0] : 1) : 1.f;
  const bool uni = smooth_mode == CCE_SMOOTH_UNIFORM;
  for (int n = blockIdx.x; n < N; n += gridDim.x) {
    const T* row = X + (long)n * ld;
    TO* drow = dX + (long)n * ldg;
    const RowSplit<T> sp(row, V);
    const long lab = load_label(labels, labels64, n);
    const bool valid = lab != ignore_index;
    const long t = (valid && lab >= 0 && lab < V) ? lab : -1;
    float tval = 0.f;
    if (tid == 0 && t >= 0) tval = elem_to_f32(row[t]);
    // pass 1: online max / sum-exp (base 2) and the row sum
    float m = kNegBig, s = 0.f, sx = 0.f;
    auto add1 = [&](float x) {
      const float x2 = x * kLog2e, mn = fmaxf(m, x2);
      s = s * fast_exp2(m - mn) + fast_exp2(x2 - mn);
      m = mn;
      sx += x;
    };
    if (tid < sp.head) add1(elem_to_f32(row[tid]));
    if (tid < V - sp.tail_start) add1(elem_to_f32(row[sp.tail_start + tid]));
    const u32x4* body = reinterpret_cast<const u32x4*>(row + sp.head);
    // ordinary loads: the lines stay in the memory-side cache for pass 2
    for_each_chunk<kFusedThreads, false>(body, sp.chunks, tid, [&](int, const u32x4& raw) {
      const T* v = reinterpret_cast<const T*>(&raw);
      float x[E], mx = kNegBig, cs = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float xe = elem_to_f32(v[e]);
        cs += xe;
        x[e] = xe * kLog2e;
        mx = fmaxf(mx, x[e]);
      }
      const float mn = fmaxf(m, mx);
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc += fast_exp2(x[e] - mn);
      s = s * fast_exp2(m - mn) + acc;
      m = mn;
      sx += cs;
    });
    block_merge_ms<NW>(m, s, red);
    if (uni) sx = block_sum<NW>(sx, red);
    const float lse = m * kLn2 + logf(s + 1e-10f);
    if (tid == 0) {
      const float smooth = uni ? lse - sx / (float)V : logV;
      const float loss = valid ? (1.f - eps) * (lse - tval) + eps * smooth + zw * lse * lse : 0.f;
      lse_out[n] = lse;
      rowloss[n] = loss;
      bsum[n] = loss;
      bcnt[n] = valid ? 1 : 0;
    }
    // pass 2: the gradient
    const float cP = valid ? g * ((uni ? 1.f : 1.f - eps) + 2.f * zw * lse) : 0.f;
    const float cU = valid && uni ? g * eps / (float)V : 0.f;
    const float cT = valid ? g * (1.f - eps) : 0.f;
    const float l2 = lse * kLog2e;
    auto grad1 = [&](int v, float x) { return (cP * fast_exp2(x * kLog2e - l2) - cU) - (v == t ? cT : 0.f); };
    if ((reinterpret_cast<uintptr_t>(drow + sp.head) & 15u) != 0) {
      for (int v = tid; v < V; v += kFusedThreads) drow[v] = f32_to_elem<TO>(grad1(v, elem_to_f32(row[v])));
    } else {
      if (tid < sp.head) drow[tid] = f32_to_elem<TO>(grad1(tid, elem_to_f32(row[tid])));
      if (tid < V - sp.tail_start) {
        const int v = sp.tail_start + tid;
        drow[v] = f32_to_elem<TO>(grad1(v, elem_to_f32(row[v])));
      }
      u32x4* dbody = reinterpret_cast<u32x4*>(drow + sp.head);
      for_each_chunk<kFusedThreads, kFusedPass2Stream>(body, sp.chunks, tid, [&](int c, const u32x4& raw) {
        const T* v = reinterpret_cast<const T*>(&raw);
        u32x4 out[kOut];
        TO* o = reinterpret_cast<TO*>(out);
        const int v0 = sp.head + c * E;
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = f32_to_elem<TO>(grad1(v0 + e, elem_to_f32(v[e])));
#pragma unroll
        for (int k = 0; k < kOut; ++k) __builtin_nontemporal_store(out[k], dbody + c * kOut + k);
      });
    }
    __syncthreads();  // red is rewritten by the next row's merge
  }
}

// Row compaction (forward with labelled rows only, and backward).  One
// workgroup partitions the rows: the rows whose label is not ignore_index go
// first, in order (idx[0 .. cnt)), the ignored ones after them (idx[cnt ..
// N), in reverse order).  live[0] = min(N, 256 * max(1, ceil(cnt / 256))):
// the row tiles the GEMMs run over; the ignored rows inside them carry zero
// coefficients (backward) or are not read back (forward).
__global__ __launch_bounds__(1024) void compact_rows_kernel(const void* labels, int labels64, int N,
                                                            long ignore_index, int* __restrict__ idx,
                                                            int* __restrict__ live, int nb_fwd, int tiles_n,
                                                            int ncu) {
  // Rounds of 16384 rows; thread t owns the 16 consecutive rows t*16 ..
  // t*16+15 of a round, packs their valid bits into a mask, and one
  // block-wide exclusive scan of the per-thread counts places them.
  constexpr int kE = 16, kRound = 1024 * kE;
  __shared__ int wv[16], wi[16];
  __shared__ int base[2];
  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
  if (tid == 0) base[0] = base[1] = 0;
  for (int r0 = 0; r0 < N; r0 += kRound) {
    const int n0 = r0 + tid * kE;
    // all 16 loads issued before any is used (indices clamped into range)
    long lab[kE];
#pragma unroll
    for (int k = 0; k < kE; ++k) lab[k] = load_label(labels, labels64, min(n0 + k, N - 1));
    unsigned mask = 0, inr = 0;
#pragma unroll
    for (int k = 0; k < kE; ++k) {
      if (n0 + k < N) {
        inr |= 1u << k;
        if (lab[k] != ignore_index) mask |= 1u << k;
      }
    }
    const int cv = __popc(mask), ci = __popc(inr & ~mask);
    // inclusive scan of (cv, ci) within the wave
    int sv = cv, si = ci;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int tv = __shfl_up(sv, o), ti = __shfl_up(si, o);
      if (l >= o) {
        sv += tv;
        si += ti;
      }
    }
    if (l == 63) {
      wv[w] = sv;
      wi[w] = si;
    }
    __syncthreads();
    int ov = base[0] + sv - cv, oi = base[1] + si - ci;  // exclusive offsets within the round
    for (int k = 0; k < w; ++k) {
      ov += wv[k];
      oi += wi[k];
    }
#pragma unroll
    for (int k = 0; k < kE; ++k) {
      if (!((inr >> k) & 1u)) continue;
      if ((mask >> k) & 1u)
        idx[ov++] = n0 + k;
      else
        idx[N - 1 - oi++] = n0 + k;
    }
    __syncthreads();
    if (tid == 0) {
      for (int k = 0; k < 16; ++k) {
        base[0] += wv[k];
        base[1] += wi[k];
      }
    }
    __syncthreads();
  }
  const int tiles = base[0] > 0 ? (base[0] + kBM - 1) / kBM : 1;
  if (tid == 0) live[0] = (int)((long)tiles * kBM < N ? (long)tiles * kBM : N);
  if (nb_fwd > 0) {
    // the forward's vocabulary splits over the live row tiles (live[1]): the
    // cheapest s of at most nb_fwd / tiles workgroups per row tile by
    // split_cost, and at least enough for 4 rounds of workgroups when the
    // launch allows (long single-round schedules leave CUs idle at the end);
    // thread t prices s = t + 1, ties go to the larger s
    const int gl = (int)((min((long)tiles * kBM, (long)N) + kBM - 1) / kBM);
    const int smax = max(1, min(min(nb_fwd / gl, tiles_n), 1024));
    const int smin = min(smax, max(1, (4 * ncu + gl - 1) / gl));
    __shared__ float cost[1024];
    __shared__ int arg[1024];
    const int sv = tid + 1;
    cost[tid] = (sv >= smin && sv <= smax) ? split_cost(gl, tiles_n, sv, ncu) : FLT_MAX;
    arg[tid] = sv;
    __syncthreads();
    for (int o = 512; o >= 1; o >>= 1) {
      if (tid < o) {
        const float c2 = cost[tid + o];
        const int a2 = arg[tid + o];
        if (c2 < cost[tid] || (c2 == cost[tid] && a2 > arg[tid])) {
          cost[tid] = c2;
          arg[tid] = a2;
        }
      }
      __syncthreads();
    }
    if (tid == 0) live[1] = arg[0];
  }
}

// out[i][:] = H[idx[i]][:] for i < N (rows of d bf16, d a multiple of 8).
__global__ __launch_bounds__(256) void gather_rows_kernel(const bf16_t* __restrict__ H, int d,
                                                          const int* __restrict__ idx, int N,
                                                          bf16_t* __restrict__ out) {
  const int chunks = d >> 3;
  const long total = (long)N * chunks;
  for (long q = blockIdx.x * 256L + threadIdx.x; q < total; q += (long)gridDim.x * 256) {
    const long i = q / chunks;
    const int c = (int)(q - i * chunks);
    *reinterpret_cast<u32x4*>(out + i * d + c * 8) =
        *reinterpret_cast<const u32x4*>(H + (long)idx[i] * d + c * 8);
  }
}

// Zero the rows idx[i], live[0] <= i < N, of a [N][d] output (row_bytes =
// d * element size, a multiple of 16): the rows no backward GEMM writes.
__global__ __launch_bounds__(256) void zero_rows_kernel(char* __restrict__ out, long row_bytes,
                                                        const int* __restrict__ idx, const int* __restrict__ live,
                                                        int N) {
  const int first = live[0];
  const long chunks = row_bytes >> 4;
  const long total = (long)(N - first) * chunks;
  for (long q = blockIdx.x * 256L + threadIdx.x; q < total; q += (long)gridDim.x * 256) {
    const long i = first + q / chunks;
    const long c = q % chunks;
    *reinterpret_cast<u32x4*>(out + (long)idx[i] * row_bytes + c * 16) = u32x4{0u, 0u, 0u, 0u};
  }
}

// The reduction of a K-split dH as a launch of its own (after the last band).
__global__ __launch_bounds__(256) void dh_reduce_kernel(DhReduce r) {
  dh_reduce_body(r, blockIdx.x * 256L + threadIdx.x, (long)gridDim.x * 256);
}

// Per-row backward coefficients, for GEMM row i of source row idx[i] (idx
// null: i).
__global__ __launch_bounds__(256) void bwd_prep_kernel(const float* __restrict__ grad_out,
                                                       const float* __restrict__ lse,
                                                       const int32_t* __restrict__ nvalid, const void* labels,
                                                       int labels64, int N, int V, long ignore_index, float eps,
                                                       float zw, int reduction, const int* __restrict__ idx,
                                                       float4* __restrict__ rowp, int* __restrict__ rowlab) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const int n = idx ? idx[i] : i;
  const long lab = load_label(labels, labels64, n);
  const bool valid = (lab != ignore_index);
  float scale = 0.f;
  if (valid) {
    const float gsc = (reduction == CCE_REDUCTION_NONE) ? grad_out[n] : grad_out[0];
    const int nv = nvalid[0];
    scale = (reduction == CCE_REDUCTION_MEAN) ? gsc / (float)(nv > 1 ? nv : 1) : gsc;
  }
  if (valid) {
    const float L = lse[n];
    rowp[i] = make_float4(L * kLog2e, scale * (1.f + 2.f * zw * L), scale * (1.f - eps), scale * eps / (float)V);
    rowlab[i] = (lab >= 0 && lab < V) ? (int)lab : -1;
  } else {
    rowp[i] = make_float4(FLT_MAX, 0.f, 0.f, 0.f);
    rowlab[i] = -1;
  }
}

// out[c][r] = in[r][c] for r < R (zero for R <= r < Rpad), c < C, over the
// 64 x 64 tile at (r0, c0), by NT threads staging through t.  With a row map,
// row r of the input is row rmap[r] of in.
template <int NT>
__device__ inline void transpose_tile(const bf16_t* __restrict__ in, long ldi, int R, int C, bf16_t* __restrict__ out,
                                      long ldo, int Rpad, int r0, int c0, bf16_t (*t)[66], int tid,
                                      const int* __restrict__ rmap) {
#pragma unroll
  for (int it = 0; it < 512 / NT; ++it) {
    const int q = tid + it * NT;         // 512 chunks of 8 elements
    const int rr = q >> 3, cc = (q & 7) * 8;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (r0 + rr < R && c0 + cc < C) {
      const long r = rmap ? (long)rmap[r0 + rr] : (long)(r0 + rr);
      v = *reinterpret_cast<const u32x4*>(in + r * ldi + c0 + cc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[rr][cc + 2 * e] = (bf16_t)(v[e] & 0xffffu);
      t[rr][cc + 2 * e + 1] = (bf16_t)(v[e] >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 512 / NT; ++it) {
    const int q = tid + it * NT;
    const int cc = q >> 3, rr = (q & 7) * 8;
    if (c0 + cc < C && r0 + rr < Rpad) {
      u32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (uint32_t)t[rr + 2 * e][cc] | ((uint32_t)t[rr + 2 * e + 1][cc] << 16);
      *reinterpret_cast<u32x4*>(out + (long)(c0 + cc) * ldo + r0 + rr) = v;
    }
  }
}

__global__ __launch_bounds__(256) void transpose_kernel(const bf16_t* __restrict__ in, long ldi, int R, int C,
                                                        bf16_t* __restrict__ out, long ldo, int Rpad,
                                                        const int* __restrict__ rmap) {
  __shared__ bf16_t t[64][66];
  transpose_tile<256>(in, ldi, R, C, out, ldo, Rpad, blockIdx.x * 64, blockIdx.y * 64, t, threadIdx.x, rmap);
}

// dB[c] = sum_m G[m][c] for c < C (fixed order: deterministic).  Block = 64
// columns.  With `live`, M = min(M, live rows of the block at live_base);
// with `accumulate`, out[c] += the sum (row blocks after the first).
__global__ __launch_bounds__(256) void colsum_kernel(const bf16_t* __restrict__ G, long ldg, int M, int C,
                                                     const int* __restrict__ live, int live_base, int accumulate,
                                                     float* __restrict__ out) {
  // blockIdx.y = row split: rows [y*M/gridDim.y, (y+1)*M/gridDim.y) into out[y][C]
  __shared__ float part[32][65];
  if (live) M = min(M, live_rows(live, live_base));
  const int tid = threadIdx.x;
  const int cg = tid & 7, rg = tid >> 3;  // 8 column groups of 8, 32 row groups
  const int c0 = blockIdx.x * 64 + cg * 8;
  const int m0 = (int)(((long)M * blockIdx.y) / gridDim.y), m1 = (int)(((long)M * (blockIdx.y + 1)) / gridDim.y);
  out += (long)blockIdx.y * C;
  float a[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = 0.f;
  if (c0 < C) {
    for (int m = m0 + rg; m < m1; m += 32) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(G + (long)m * ldg + c0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[2 * e] += bf16_to_f32(v[e] & 0xffffu);
        a[2 * e + 1] += bf16_to_f32(v[e] >> 16);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) part[rg][cg * 8 + e] = a[e];
  __syncthreads();
  if (tid < 64) {
    float s = 0.f;
    for (int r = 0; r < 32; ++r) s += part[r][tid];
    const int c = blockIdx.x * 64 + tid;
    if (c < C) out[c] = accumulate ? out[c] + s : s;
  }
}

// out[c] = sum over r of part[r][c] in order r = 0..R-1; block 0 also writes
// out[C] = sum of vec[0..n) (fixed-order tree), or 0 without vec.
__global__ __launch_bounds__(256) void sum_parts_kernel(const float* __restrict__ part, int R, int C,
                                                        const float* __restrict__ vec, int n,
                                                        float* __restrict__ out) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c < C) {
    float s = 0.f;
    for (int r = 0; r < R; ++r) s += part[(long)r * C + c];
    out[c] = s;
  }
  if (blockIdx.x == 0) {
    __shared__ float red[256];
    float a = 0.f;
    if (vec)
      for (int i = threadIdx.x; i < n; i += 256) a += vec[i];
    red[threadIdx.x] = a;
    __syncthreads();
    for (int o = 128; o >= 1; o >>= 1) {
      if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
      __syncthreads();
    }
    if (threadIdx.x == 0) out[C] = red[0];
  }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t* __restrict__ p, long nwords) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nwords; i += (long)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

#define HIP_TRY(expr)                                                                         \
  do {                                                                                        \
    hipError_t e_ = (expr);                                                                   \
    if (e_ != hipSuccess) return fail(CCE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
inline long ceil_div(long a, long b) { return (a + b - 1) / b; }

struct Carver {
  char* base;
  size_t off = 0;
  explicit Carver(void* p) : base(static_cast<char*>(p)) {}
  template <class T>
  T* take(size_t count) {
    off = align_up(off, 256);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

// Forward vocabulary splits: enough (row tile x split) workgroups to cover
// the 256 CUs several times over.
bool fast_k(long K) { return K % 64 == 0; }
int lse_bn(long d) { return fast_k(d) ? kFastBN : kSlowBN; }

// Vocabulary splits per row tile of a forward over every row tile: about 512
// workgroups for few row tiles (runs of several vocabulary tiles, so the
// pipeline's start is paid once per run), never fewer splits than
// min(32, 2048 / row tiles): large batches keep their split counts.
int forward_splits(long N, long d, long V) {
  if (N <= 0) return 1;
  const long gm = ceil_div(N, kBM), tn = ceil_div(V, lse_bn(d));
  long s = std::max(ceil_div(512, gm), std::min<long>(32, ceil_div(2048, gm)));
  if (s > tn) s = tn;
  if (s < 1) s = 1;
  return (int)s;
}

// Workgroups of the forward GEMM, each with a slot of 256 rows of (max,
// sum-exp) partials.  A forward over every row tile runs forward_splits per
// row tile.  A compacted forward re-splits the vocabulary over the live row
// tiles on the device (compact_rows_kernel picks the count by split_cost,
// within the launch's workgroups): it launches room for up to 64 splits per
// row tile (short workgroups, so the partly filled last round left when some
// row tiles drop out costs little), but no more than 8192 workgroups beyond
// the count over every row tile, which bounds its partials at large N
// (16 MiB at N = 2^21 rather than 1 GiB).
long forward_slots(long N, long d, long V, bool compact) {
  const long gm = ceil_div(std::max<long>(N, 1), kBM);
  const long base = gm * forward_splits(N, d, V);
  if (!compact) return base;
  const long tn = ceil_div(V, lse_bn(d));
  return std::max(base, std::min(gm * std::min<long>(64, tn), 8192L));
}

// CUs of the current device (cached per device).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Vocabulary band width: chunk rounded up to a multiple of 256, at most
// kBandCap (8192) columns and at least 256, within V rounded up.  chunk_size
// bounds the band from above only: the reference's trainer asks for 16384 at
// V >= 128K (get_optimal_chunk_size), which here would double the band
// buffers for no measured gain.
constexpr long kMaxBand = 1L << 20;
constexpr long kBandCap = 8192;
long band_width(long V, long chunk, long N, long d) {
  long vb = chunk <= 0 ? kBandCap : std::min(chunk, kBandCap);
  vb = align_up((size_t)vb, 256);
  // with few rows a band launch is short and its fixed costs dominate: up to
  // 4x wider bands, while the band buffers (G: rows x band, W^T: d x band)
  // stay within what 4096 rows take at that band.  Below 1024 rows W^T and
  // the dH partials would outgrow the logits themselves, for no measured gain.
  const long rows = (long)align_up((size_t)(N > 0 ? N : 1), 256);
  const long f = rows < 1024 ? 1 : std::min<long>(4, std::max<long>(1, (4096 + d) / (rows + d)));
  vb = std::min<long>(vb * f, kMaxBand);
  const long vmax = (long)align_up((size_t)V, 256);
  if (vb > vmax) vb = vmax;
  if (vb < 256) vb = 256;
  return vb;
}

// Rows per block of the backward.  The band gradient G of a block is
// (rows x band) bf16 and there are two such buffers (band b+1's recompute
// overlaps band b's GEMMs), so a block has at most budget / (4 * band) rows,
// a multiple of 256; a batch that fits is one block.  G's memory is then
// bounded by the budget whatever N is; dW of a band accumulates over the
// blocks.  The budget is 512 MiB, or CHRONICALS_CCE_G_BUDGET_MB from the
// environment (read on every call, so a workspace query and the call it
// sizes must see the same value).
constexpr long kGBudget = 512L << 20;
long g_budget() {
  const char* e = getenv("CHRONICALS_CCE_G_BUDGET_MB");
  if (e && *e) {
    const long mb = strtol(e, nullptr, 10);
    if (mb > 0 && mb < (1L << 20)) return mb << 20;
  }
  return kGBudget;
}
long block_rows(long N, long Vb) {
  const long n = std::max<long>(N, 1);
  long nb = g_budget() / (4 * Vb) / kBM * kBM;
  if (nb < kBM) nb = kBM;
  return nb >= n ? n : nb;
}

// The compacted GEMMs take H's rows either from a gathered copy (Hc, N x d
// bf16 of workspace, written by gather_rows_kernel) or straight from H
// through the row order (ARows).  Reading through the order costs each
// workgroup a dependent load before its first slab (about 1.5% of a C2 band
// launch, whose recompute workgroups run one tile each), so the copy is kept
// while it is small next to the band state (H below 256 MiB); from there up
// to the DMA's 32-bit lane offsets (2 GiB) the rows are read in place, and
// past that the copy returns.  `prefer` (the forward without a workspace,
// whose scratch is fixed) reads in place wherever the offsets allow.
// CHRONICALS_CCE_ROW_GATHER=0 forces the copy, =1 reads in place wherever the
// offsets allow (read on every call, so a workspace query and the call it
// sizes must see the same value).
constexpr long kInPlaceMinBytes = 256L << 20;
bool rows_in_place(long N, long d, bool prefer = false) {
  const long bytes = N * d * 2;
  if (bytes > 0x7ffffff0L) return false;
  const char* e = getenv("CHRONICALS_CCE_ROW_GATHER");
  if (e && (e[0] == '0' || e[0] == '1') && e[1] == 0) return e[0] == '1';
  return prefer || bytes >= kInPlaceMinBytes;
}

struct FwdLayout {
  float *pm, *ps, *bsum, *rowloss;
  int* bcnt;
  float *wpart, *wsum;  // column sums of W by row split, and their total (+ the bias sum)
  int wsplits;
  // row compaction (CCE_LSE_LABELLED_ROWS, d a multiple of 64): row order,
  // live row count, and H in that order when the GEMM cannot read H through
  // the row order
  int* idx;
  int* live;
  bf16_t* Hc;
  size_t bytes;
};

// Row splits of the column sum of W: enough workgroups to stream W, at most
// 2^22 partial floats.
int wsum_splits(long d, long V) {
  long r = (1L << 22) / (d > 0 ? d : 1);
  r = r < 1 ? 1 : (r > 64 ? 64 : r);
  const long rows = ceil_div(V, 256);
  return (int)(r < rows ? r : (rows > 0 ? rows : 1));
}

// The forward compacts its rows when only the labelled rows' lse is wanted
// and the direct-to-LDS GEMM runs (d a multiple of 64).
bool fwd_compacts(long d, int lse_rows) { return lse_rows == CCE_LSE_LABELLED_ROWS && fast_k(d); }

FwdLayout fwd_layout(void* ws, long N, long d, long V, int reduction, int lse_rows, bool prefer_in_place = false) {
  Carver c(ws);
  FwdLayout L;
  const bool compact = fwd_compacts(d, lse_rows) && N > 0;
  const long nb = ceil_div(N, 4);
  // [S][N rounded up to 256] partials, or for a compacted forward one slot of
  // 256 rows per launched workgroup
  const size_t parts = (size_t)forward_slots(N, d, V, compact) * kBM;
  L.pm = c.take<float>(parts);
  L.ps = c.take<float>(parts);
  L.bsum = c.take<float>((size_t)(nb > 0 ? nb : 1));
  L.bcnt = c.take<int>((size_t)(nb > 0 ? nb : 1));
  L.rowloss = (reduction == CCE_REDUCTION_NONE) ? nullptr : c.take<float>((size_t)(N > 0 ? N : 1));
  L.wsplits = wsum_splits(d, V);
  L.wpart = c.take<float>((size_t)L.wsplits * d);
  L.wsum = c.take<float>((size_t)d + 1);
  L.idx = compact ? c.take<int>((size_t)N) : nullptr;
  L.live = compact ? c.take<int>(2) : nullptr;  // live rows, vocabulary splits
  L.Hc = compact && !rows_in_place(N, d, prefer_in_place) ? c.take<bf16_t>((size_t)N * d) : nullptr;
  L.bytes = align_up(c.off, 256);
  return L;
}

struct BwdLayout {
  long N;        // rows
  long Vb, Nb;    // band width, rows per block
  int nblocks;    // row blocks
  float4* rowp;
  int* rowlab;
  bf16_t* G[2];   // band gradient of a block; the second only when units alternate
  bf16_t* WT[2];  // W band transposes; the second only when bands alternate
  bf16_t* HT;
  // Caller output memory that is not yet written doubles as scratch (banded
  // backward, bf16 dH and dW wanted, several bands):
  //  - ht_out: H^T ([d][N], N a multiple of 64) lives in grad_hidden, which
  //    the bands leave unwritten: the last band adds into the fp32 dH
  //    accumulator, and dH goes to grad_hidden after the last band launch;
  //  - wt_out: W^T of band b lives in the rows of band b + 1 of grad_weight,
  //    which dW writes only in band b + 1.  The last band's W^T takes WT[0],
  //    or, when dW accumulates over row blocks in dWacc (wt_last_in_place),
  //    the last band's own rows of grad_weight, whose dW is then written
  //    after the last band launch;
  //  - wt_dh (no dW wanted, N >= 2 * Vb): both W^T buffers live in
  //    grad_hidden.
  // dh_late = ht_out || wt_dh: dH is written after the last band launch.
  bool ht_out, wt_out, wt_last_in_place, wt_dh, dh_late;
  float* dHacc;   // dH over the bands (bf16 dH with several bands; fp32 dH accumulates in place)
  float* dWacc;   // dW of a band over the row blocks (bf16 dW with several blocks)
  // row compaction (banded backward): row order, live row count, and H in
  // that order when the GEMMs cannot read H through the row order
  int* idx;
  int* live;
  bf16_t* Hc;
  // fp32 partials of a K-split dH: dh_ks slices of [Nb][d] per unit, in two
  // alternating buffers when the reduction is folded into the next launch;
  // null when unsplit
  float* dhpart;
  int dh_ks;
  size_t bytes;
};

// The banded backward with the band kernel (d a multiple of 64) overlaps the
// recompute of band b+1 with the dW / dH GEMMs of band b: two G buffers.
bool banded(long d) { return d % 64 == 0; }

// Hidden columns of the banded backward's 256-wide dW / dH tiles; the rest,
// when d % 256 <= 128, is one 128-wide tail tile.
long band_dmain(long d) { return (d % 256 == 0 || d % 256 > 128) ? d : d - d % 256; }

// With 4 or more K splits (very few rows) the band launches are short, and
// each band's dH reduction rides in the next band's launch (two partial
// buffers, alternating); with 2-3 splits it is a launch of its own.
bool dh_fold(int ks) { return ks >= 4; }

// K splits of the banded dH.  dH has one tile per (256-row tile, hidden
// column tile), each reducing over the whole band; with few rows those tiles
// cannot fill the CUs and the band launch waits on their long K loops.  Then
// K is split so that tiles x splits reaches about 128 workgroups, with at
// least 8 slabs of 64 per split (more splits cost more in the fp32 partials'
// reduction than their shorter K loops return).
int dh_splits(long N, long d, long Vb) {
  if (!banded(d) || N <= 0 || d <= 0) return 1;
  const long dmain = band_dmain(d);
  const long tiles = ceil_div(N, kBM) * (ceil_div(dmain, kFastBN) + (dmain < d ? 1 : 0));
  if (tiles <= 0 || tiles >= 128) return 1;
  const long ks = std::min<long>(ceil_div(128, tiles), Vb / 512);
  return ks < 2 ? 1 : (int)ks;
}

// Columns of H^T ([d][N] as dW's K-major B operand): N rounded up to whole
// 64-wide slabs, the padding zeroed by the transpose, so every slab of the
// dW reduction lies inside a row of H^T (kmajor_fits).
long ht_cols(long N) { return (long)align_up((size_t)N, kBK); }

BwdLayout bwd_layout(void* ws, long N, long d, long V, long Vb, bool need_dh, bool need_dw, bool dh_f32,
                     bool dw_f32) {
  Carver c(ws);
  BwdLayout L;
  L.N = N;
  L.Vb = Vb;
  L.Nb = block_rows(N, Vb);
  L.nblocks = (int)ceil_div(std::max<long>(N, 1), L.Nb);
  const long nbands = ceil_div(V, Vb);
  const long units = nbands * L.nblocks;
  const long N64 = ht_cols(N);
  L.rowp = c.take<float4>((size_t)N);
  L.rowlab = c.take<int>((size_t)N);
  L.ht_out = banded(d) && need_dh && need_dw && !dh_f32 && nbands > 1 && N % 64 == 0;
  L.wt_out = banded(d) && need_dh && need_dw && nbands > 1;
  L.wt_last_in_place = L.wt_out && L.nblocks > 1 && !dw_f32;
  L.wt_dh = banded(d) && need_dh && !need_dw && !dh_f32 && nbands > 1 && N >= 2 * Vb;
  L.dh_late = L.ht_out || L.wt_dh;
  L.G[0] = c.take<bf16_t>((size_t)L.Nb * Vb);
  L.G[1] = (banded(d) && units > 1) ? c.take<bf16_t>((size_t)L.Nb * Vb) : L.G[0];
  L.WT[0] = need_dh && !L.wt_last_in_place && !L.wt_dh ? c.take<bf16_t>((size_t)d * Vb) : nullptr;
  L.WT[1] = (need_dh && banded(d) && nbands > 1 && !L.wt_out && !L.wt_dh) ? c.take<bf16_t>((size_t)d * Vb)
                                                                          : L.WT[0];
  L.HT = need_dw && !L.ht_out ? c.take<bf16_t>((size_t)d * N64) : nullptr;
  L.dHacc = (need_dh && nbands > 1 && !dh_f32) ? c.take<float>((size_t)N * d) : nullptr;
  L.dWacc = (need_dw && L.nblocks > 1 && !dw_f32) ? c.take<float>((size_t)Vb * d) : nullptr;
  const bool compact = banded(d);
  L.idx = compact ? c.take<int>((size_t)N) : nullptr;
  L.live = compact ? c.take<int>(1) : nullptr;
  L.Hc = compact && !rows_in_place(N, d) ? c.take<bf16_t>((size_t)N * d) : nullptr;
  L.dh_ks = need_dh ? dh_splits(L.Nb, d, Vb) : 1;
  // a second partial buffer only when the reduction rides in the next
  // launch (dh_fold); otherwise each unit's reduction runs before the next
  // band launch writes the one buffer again
  L.dhpart = L.dh_ks > 1 ? c.take<float>((size_t)(dh_fold(L.dh_ks) && units > 1 ? 2 : 1) * L.dh_ks * L.Nb * d)
                         : nullptr;
  L.bytes = align_up(c.off, 256);
  return L;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

// The direct-to-LDS pipelines read K-major operands in 64-wide slabs with the
// slab's k offset outside the buffer range check (dma_kmajor), so each
// operand row must hold every slab the GEMM reads: kb + K rounded up to 64
// columns at most ld.  Checked on the host before each launch; a layout that
// broke it would otherwise read past the operand.
bool kmajor_fits(long ld, long kb, long K) { return K <= 0 || kb + (long)align_up((size_t)K, kBK) <= ld; }
int check_kmajor(const GemmShape& g, bool a_kmajor) {
  if ((a_kmajor && !kmajor_fits(g.lda, 0, g.K)) || !kmajor_fits(g.ldb, g.kb, g.K))
    return fail(CCE_ERR_INVALID_ARG, "internal: a K-major operand row (lda %ld, ldb %ld) is shorter than the "
                "slabs of K = %d at k offset %d", g.lda, g.ldb, g.K, g.kb);
  return CCE_OK;
}

constexpr long kMaxRows = 1L << 21;  // tokens per call

int check_dims(long N, long d, long V) {
  if (N < 0) return fail(CCE_ERR_INVALID_ARG, "N must be >= 0 (got %ld)", N);
  if (d <= 0 || d % 8 != 0) return fail(CCE_ERR_INVALID_ARG, "hidden dim d must be a positive multiple of 8 (got %ld)", d);
  if (V <= 0) return fail(CCE_ERR_INVALID_ARG, "vocab size V must be > 0 (got %ld)", V);
  // N: the dW GEMM reads 256-row tiles of H^T ([d][N]) through one buffer
  // descriptor, whose range (2 GB) and 32-bit lane offsets bound 256*N*2 bytes
  if (N > kMaxRows || V > (1L << 30) || d > (1L << 20))
    return fail(CCE_ERR_INVALID_ARG, "problem too large (N=%ld d=%ld V=%ld; limits N <= %ld, V <= 2^30, d <= 2^20)",
                N, d, V, kMaxRows);
  return CCE_OK;
}

// Optional per-kind kernel timing (cce_kernel_timing_enable).
struct TimedLaunch {
  hipEvent_t ev0, ev1;
  double credited, executed;  // algorithmic / executed MFMA FLOPs of the launch
};
struct KernelTiming {
  std::mutex mu;
  bool enabled = false;
  std::vector<TimedLaunch> pending[CCE_KERNEL_KINDS];
  std::vector<hipEvent_t> pool;
  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
KernelTiming g_timing;

// Records the start event of a timed launch; returns false when timing is off.
bool timing_begin(hipStream_t st, hipEvent_t* ev0, hipEvent_t* ev1) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  if (!g_timing.enabled) return false;
  *ev0 = g_timing.get();
  *ev1 = g_timing.get();
  if (!*ev0 || !*ev1) return false;
  return hipEventRecord(*ev0, st) == hipSuccess;
}

void timing_end(int kind, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1, double credited, double executed) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  if (hipEventRecord(ev1, st) == hipSuccess) g_timing.pending[kind].push_back({ev0, ev1, credited, executed});
}

// MFMA FLOPs of an M x N x K GEMM
double gemm_flops(long M, long N, long K) { return 2.0 * (double)M * (double)N * (double)K; }

// A GEMM launch; `credited` is the algorithmic share of its FLOPs (the
// logits recompute of the backward is executed but not credited).
template <int BN, int W, bool AK, bool BK, template <int, int> class EpiT, int PIPE = 3, int NST = 2,
          bool AROW = false>
int launch_gemm(const GemmShape& g, const typename EpiT<BN, W>::Params& ep, int nblocks, hipStream_t st,
                int kind, bool credited) {
  if (nblocks <= 0) return CCE_OK;
  if (PIPE >= 4) {
    const int rc = check_kmajor(g, AK);
    if (rc) return rc;
  }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  const bool timed = timing_begin(st, &e0, &e1);
  hipLaunchKernelGGL((gemm_kernel<BN, W, AK, BK, EpiT, PIPE, NST, AROW>), dim3(nblocks), dim3(W * 64), 0, st, g, ep);
  HIP_TRY(hipGetLastError());
  if (timed) {
    const double f = gemm_flops(g.M, g.N, g.K);
    timing_end(kind, st, e0, e1, credited ? f : 0.0, f);
  }
  return CCE_OK;
}

int zero_fill(void* p, size_t bytes, hipStream_t st) {
  if (!p || bytes == 0) return CCE_OK;
  const long words = (long)(bytes / 4);
  long blocks = ceil_div(words, 256);
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, reinterpret_cast<uint32_t*>(p),
                     words);
  HIP_TRY(hipGetLastError());
  return CCE_OK;
}


int launch_dual_acc(const GemmShape& g_dw, const AccParams& e_dw, const GemmShape& g_dh, const AccParams& e_dh,
                    hipStream_t st) {
  // dH operands are K-major with K a multiple of 64 (the band is zero-padded);
  // dW reads G transposed from LDS (its K tail reads as zero past row N)
  constexpr int kBNdw = kSlowBN, kBNdh = kFastBN;
  const int nb_dw = (int)(ceil_div(g_dw.M, kBM) * ceil_div(g_dw.N, kBNdw));
  const int nb_dh = (int)(ceil_div(g_dh.M, kBM) * ceil_div(g_dh.N, kBNdh));
  if (nb_dw + nb_dh <= 0) return CCE_OK;
  int rc = nb_dw ? check_kmajor(g_dw, false) : CCE_OK;
  if (!rc && nb_dh) rc = check_kmajor(g_dh, true);
  if (rc) return rc;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  const bool timed = timing_begin(st, &t0, &t1);
  hipLaunchKernelGGL((dual_acc_kernel<kWarp8, kBNdw, 5, kBNdh, 4>), dim3(nb_dw + nb_dh), dim3(kWarp8 * 64), 0, st,
                     g_dw, e_dw, nb_dw, g_dh, e_dh);
  HIP_TRY(hipGetLastError());
  if (timed) {
    const double f = gemm_flops(g_dw.M, g_dw.N, g_dw.K) + gemm_flops(g_dh.M, g_dh.N, g_dh.K);
    timing_end(CCE_KERNEL_BWD_DHDW, st, t0, t1, f, f);
  }
  return CCE_OK;
}

template <int BN, bool AK, int PIPE>
int launch_acc(const GemmShape& g, const AccParams& ep, hipStream_t st, int kind) {
  const int nb = (int)(ceil_div(g.M, kBM) * ceil_div(g.N, BN));
  return launch_gemm<BN, kWarp8, AK, true, EpiAcc, PIPE>(g, ep, nb, st, kind, true);
}

// Recompute launch shape of one unit: G[n][c] for the rows [m0, m0 + rows)
// of the compacted order (a row block) and columns [v0, v0 + vb).
// A recompute launch of its own runs one round of workgroups, about one per
// CU, each over a run of column tiles: the pipeline runs on across a run, so
// a tile's epilogue overlaps the next tile's first loads, and no partly filled
// last round is left.  Inside the band launch (`in_band`) each workgroup
// takes one tile, the finest grain for filling the CUs that the long dW / dH
// tiles leave idle.
void grad_shape(const bf16_t* H, const bf16_t* W, const float* bias, const BwdLayout& L, bf16_t* G, long m0,
                long rows, long d, long v0, long vb, int bn, bool in_band, GemmShape& g, GradParams& e, int& nb) {
  const int gm = (int)ceil_div(rows, kBM);
  if (L.Hc || !L.idx) {
    g.A = (L.Hc ? L.Hc : H) + m0 * d;
  } else {
    g.A = H;
    g.arow = L.idx + m0;
    g.arows = L.N;
  }
  g.lda = d; g.B = W + v0 * d; g.ldb = d;
  g.M = (int)rows; g.N = (int)vb; g.K = (int)d;
  g.live = L.live; g.dyn = L.live ? kDynM : kDynNone; g.live_base = (int)m0;
  e.bias = bias; e.rowp = L.rowp + m0; e.rowlab = L.rowlab + m0; e.G = G; e.ldg = L.Vb; e.v0 = (int)v0;
  e.tiles_n = (int)ceil_div(vb, bn);
  e.splits = in_band ? e.tiles_n : (int)std::min<long>(e.tiles_n, std::max<long>(1, ceil_div(device_cus(), gm)));
  nb = gm * e.splits;
}

int launch_band(const BandLaunch& p, bool has_bias, hipStream_t st, int kind = CCE_KERNEL_BWD_BAND) {
  const int nb = p.nb_dw + p.nb_dw2 + p.nb_dh + p.nb_dh2 + p.nb_gr + p.nb_red + p.nb_tr;
  if (nb <= 0) return CCE_OK;
  int rc = CCE_OK;
  if (p.nb_dw) rc = check_kmajor(p.dw, false);
  if (!rc && p.nb_dw2) rc = check_kmajor(p.dw2, false);
  if (!rc && p.nb_dh) rc = check_kmajor(p.dh, true);
  if (!rc && p.nb_dh2) rc = check_kmajor(p.dh2, true);
  if (!rc && p.nb_gr) rc = check_kmajor(p.gr, true);
  if (rc) return rc;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  const bool timed = timing_begin(st, &t0, &t1);
  const bool arow = p.gr.arow != nullptr;
  if (has_bias && arow)
    hipLaunchKernelGGL((band_kernel<true, true>), dim3(nb), dim3(kWarp8 * 64), 0, st, p);
  else if (has_bias)
    hipLaunchKernelGGL((band_kernel<true, false>), dim3(nb), dim3(kWarp8 * 64), 0, st, p);
  else if (arow)
    hipLaunchKernelGGL((band_kernel<false, true>), dim3(nb), dim3(kWarp8 * 64), 0, st, p);
  else
    hipLaunchKernelGGL((band_kernel<false, false>), dim3(nb), dim3(kWarp8 * 64), 0, st, p);
  HIP_TRY(hipGetLastError());
  if (timed) {
    double cr = 0.0;
    if (p.nb_dw) cr += gemm_flops(p.dw.M, p.dw.N, p.dw.K);
    if (p.nb_dw2) cr += gemm_flops(p.dw2.M, p.dw2.N, p.dw2.K);
    if (p.nb_dh) cr += gemm_flops(p.dh.M, p.dh.N, p.dh.K);
    if (p.nb_dh2) cr += gemm_flops(p.dh2.M, p.dh2.N, p.dh2.K);
    const double ex = cr + (p.nb_gr ? gemm_flops(p.gr.M, p.gr.N, p.gr.K) : 0.0);
    timing_end(kind, st, t0, t1, cr, ex);
  }
  return CCE_OK;
}

// Logits-in cross-entropy: dtype codes and workspace.
int logits_elem_size(int dtype) {
  return dtype == CCE_DTYPE_F32 ? 4 : (dtype == CCE_DTYPE_BF16 || dtype == CCE_DTYPE_F16) ? 2 : 0;
}

struct LogitsLayout {
  float *rowloss, *bsum;
  int* bcnt;
  size_t bytes;
};

LogitsLayout logits_layout(void* ws, long N) {
  Carver c(ws);
  LogitsLayout L;
  const size_t n = (size_t)(N > 0 ? N : 1);
  L.rowloss = c.take<float>(n);
  L.bsum = c.take<float>(n);
  L.bcnt = c.take<int>(n);
  L.bytes = align_up(c.off, 256);
  return L;
}

int check_logits_args(long N, long V, int dtype, long ld, int reduction, float eps, int smooth) {
  if (N < 0 || N > kMaxRows) return fail(CCE_ERR_INVALID_ARG, "N must be in [0, %ld] (got %ld)", kMaxRows, N);
  if (V <= 0 || V > (1L << 30)) return fail(CCE_ERR_INVALID_ARG, "vocab size V must be in [1, 2^30] (got %ld)", V);
  if (!logits_elem_size(dtype))
    return fail(CCE_ERR_INVALID_ARG, "logits dtype must be CCE_DTYPE_BF16, CCE_DTYPE_F16 or CCE_DTYPE_F32");
  if (ld < V) return fail(CCE_ERR_INVALID_ARG, "row stride %ld is smaller than V = %ld", ld, V);
  if (reduction < CCE_REDUCTION_NONE || reduction > CCE_REDUCTION_SUM)
    return fail(CCE_ERR_INVALID_ARG, "reduction must be 0 (none), 1 (mean) or 2 (sum), got %d", reduction);
  if (!(eps >= 0.f && eps <= 1.f)) return fail(CCE_ERR_INVALID_ARG, "label_smoothing must be in [0, 1]");
  if (smooth != CCE_SMOOTH_LOGV && smooth != CCE_SMOOTH_UNIFORM)
    return fail(CCE_ERR_INVALID_ARG, "smoothing_form must be CCE_SMOOTH_LOGV or CCE_SMOOTH_UNIFORM, got %d", smooth);
  return CCE_OK;
}

int forward_run(const void* hidden, const void* weight, const void* labels, int labels_int64, const float* bias,
                int64_t N, int64_t d, int64_t V, int64_t ignore_index, float label_smoothing, float z_loss_weight,
                int smoothing_form, int reduction, int lse_rows, float* loss_out, float* lse_out, float* target_out,
                int32_t* n_valid_out, void* workspace, size_t workspace_bytes, void* stream,
                bool prefer_in_place = false) {
  int rc = check_dims(N, d, V);
  if (rc) return rc;
  if (smoothing_form != CCE_SMOOTH_LOGV && smoothing_form != CCE_SMOOTH_UNIFORM)
    return fail(CCE_ERR_INVALID_ARG, "smoothing_form must be CCE_SMOOTH_LOGV or CCE_SMOOTH_UNIFORM, got %d",
                smoothing_form);
  if (reduction < CCE_REDUCTION_NONE || reduction > CCE_REDUCTION_SUM)
    return fail(CCE_ERR_INVALID_ARG, "reduction must be 0 (none), 1 (mean) or 2 (sum), got %d", reduction);
  if (lse_rows != CCE_LSE_ALL_ROWS && lse_rows != CCE_LSE_LABELLED_ROWS)
    return fail(CCE_ERR_INVALID_ARG, "lse_rows must be CCE_LSE_ALL_ROWS or CCE_LSE_LABELLED_ROWS, got %d", lse_rows);
  if (!n_valid_out || (!loss_out && !(reduction == CCE_REDUCTION_NONE && N == 0)))
    return fail(CCE_ERR_INVALID_ARG, "loss_out and n_valid_out must not be null");
  if (N > 0 && (!hidden || !weight || !labels || !lse_out))
    return fail(CCE_ERR_INVALID_ARG, "hidden, weight, labels and lse_out must not be null");
  if (!(label_smoothing >= 0.f && label_smoothing <= 1.f))
    return fail(CCE_ERR_INVALID_ARG, "label_smoothing must be in [0, 1]");
  if (misaligned(hidden) || misaligned(weight) || misaligned(workspace))
    return fail(CCE_ERR_INVALID_ARG, "hidden, weight and workspace must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const FwdLayout need = fwd_layout(nullptr, N, d, V, reduction, lse_rows, prefer_in_place);
  if (workspace_bytes < need.bytes || (need.bytes && !workspace))
    return fail(CCE_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need.bytes, workspace_bytes);
  if (N == 0) {
    rc = zero_fill(n_valid_out, sizeof(int32_t), st);
    if (!rc && reduction != CCE_REDUCTION_NONE) rc = zero_fill(loss_out, sizeof(float), st);
    return rc;
  }
  const FwdLayout L = fwd_layout(workspace, N, d, V, reduction, lse_rows, prefer_in_place);
  const int S = forward_splits(N, d, V);
  const int slots = (int)forward_slots(N, d, V, L.idx != nullptr);  // workgroups

  // CCE_LSE_LABELLED_ROWS: the labelled rows go first and the GEMM runs only
  // over the row tiles that hold them (the partials then follow that order)
  if (L.idx) {
    hipLaunchKernelGGL(compact_rows_kernel, dim3(1), dim3(1024), 0, st, labels, labels_int64, (int)N,
                       (long)ignore_index, L.idx, L.live, slots, (int)ceil_div(V, lse_bn(d)), device_cus());
    HIP_TRY(hipGetLastError());
    if (L.Hc) {
      const long chunks = (long)N * (d / 8);
      hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)std::min<long>(ceil_div(chunks, 256), 8192)), dim3(256),
                         0, st, static_cast<const bf16_t*>(hidden), (int)d, L.idx, (int)N, L.Hc);
      HIP_TRY(hipGetLastError());
    }
  }

  GemmShape g;
  g.A = L.Hc ? L.Hc : static_cast<const bf16_t*>(hidden);
  if (L.idx && !L.Hc) {
    g.arow = L.idx;
    g.arows = N;
  }
  g.lda = d;
  g.B = static_cast<const bf16_t*>(weight);
  g.ldb = d;
  g.M = (int)N;
  g.N = (int)V;
  g.K = (int)d;
  g.live = L.live;
  g.dyn = L.live ? kDynM : kDynNone;
  LseParams ep;
  ep.bias = bias;
  ep.pm = L.pm;
  ep.ps = L.ps;
  ep.ldp = N;
  ep.splits = S;
  ep.tiles_n = (int)ceil_div(V, lse_bn(d));
  if (fast_k(d) && g.arow)
    rc = bias ? launch_gemm<kFastBN, kWarp8, true, true, EpiLseBias, 4, 2, true>(g, ep, slots, st,
                                                                                CCE_KERNEL_FWD_LSE, true)
              : launch_gemm<kFastBN, kWarp8, true, true, EpiLse, 4, 2, true>(g, ep, slots, st, CCE_KERNEL_FWD_LSE,
                                                                            true);
  else if (fast_k(d))
    rc = bias ? launch_gemm<kFastBN, kWarp8, true, true, EpiLseBias, 4>(g, ep, slots, st, CCE_KERNEL_FWD_LSE, true)
              : launch_gemm<kFastBN, kWarp8, true, true, EpiLse, 4>(g, ep, slots, st, CCE_KERNEL_FWD_LSE, true);
  else
    rc = bias ? launch_gemm<kSlowBN, kWarp8, true, true, EpiLseBias, 3>(g, ep, slots, st, CCE_KERNEL_FWD_LSE, true)
              : launch_gemm<kSlowBN, kWarp8, true, true, EpiLse, 3>(g, ep, slots, st, CCE_KERNEL_FWD_LSE, true);
  if (rc) return rc;

  const bool uniform = smoothing_form == CCE_SMOOTH_UNIFORM && label_smoothing > 0.f;
  if (uniform) {
    hipLaunchKernelGGL(colsum_kernel, dim3((unsigned)ceil_div(d, 64), (unsigned)L.wsplits), dim3(256), 0, st,
                       static_cast<const bf16_t*>(weight), (long)d, (int)V, (int)d, nullptr, 0, 0, L.wpart);
    HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(sum_parts_kernel, dim3((unsigned)ceil_div(d, 256)), dim3(256), 0, st, L.wpart, L.wsplits,
                       (int)d, bias, (int)V, L.wsum);
    HIP_TRY(hipGetLastError());
  }
  const int nb = (int)ceil_div(N, 4);
  float* rowloss = (reduction == CCE_REDUCTION_NONE) ? loss_out : L.rowloss;
  const float logV = logf((float)V);
  hipLaunchKernelGGL(fwd_combine_kernel, dim3(nb), dim3(256), 0, st, L.pm, L.ps, S,
                     static_cast<const bf16_t*>(hidden), static_cast<const bf16_t*>(weight), labels, labels_int64,
                     bias, (int)N, (int)d, (int)V, (long)ignore_index, label_smoothing, z_loss_weight, logV,
                     uniform ? L.wsum : nullptr, lse_rows == CCE_LSE_LABELLED_ROWS, L.idx, L.live, slots,
                     ep.tiles_n, lse_out, target_out, rowloss, L.bsum, L.bcnt);
  HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(fwd_finalize_kernel, dim3(1), dim3(1024), 0, st, L.bsum, L.bcnt, nb, reduction, loss_out,
                     n_valid_out);
  HIP_TRY(hipGetLastError());
  return CCE_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Static scratch of cce_forward_noalloc: the forward's workspace for callers
// that cannot allocate device memory.  Each device that runs the library holds
// its own copy of this array (CCE_NOALLOC_SCRATCH_BYTES) until the process
// ends.  In host code `scratch` names a host-side stand-in, not device memory:
// the device address comes from hipGetSymbolAddress, once per device, and only
// that address is passed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[CCE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device and kept).
int noalloc_scratch(void** out) {
  int dev = -1;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(CCE_ERR_INVALID_ARG, "device ordinal %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(CCE_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address on device %d", dev);
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return CCE_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" {

const char* cce_last_error(void) { return g_err; }

int cce_abi_version(void) { return CCE_ABI_VERSION; }

// The build passes the SHA-256 of this file and the header as bare hex digits.
#ifndef CCE_SOURCE_HASH
#define CCE_SOURCE_HASH unknown
#endif
#define CCE_STR2(x) #x
#define CCE_STR(x) CCE_STR2(x)
const char* cce_source_hash(void) { return CCE_STR(CCE_SOURCE_HASH); }

int cce_forward_workspace_bytes(int64_t N, int64_t d, int64_t V, int reduction, int lse_rows, size_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return fail(CCE_ERR_INVALID_ARG, "bytes must not be null");
  int rc = check_dims(N, d, V);
  if (rc) return rc;
  if (reduction < CCE_REDUCTION_NONE || reduction > CCE_REDUCTION_SUM)
    return fail(CCE_ERR_INVALID_ARG, "reduction must be 0 (none), 1 (mean) or 2 (sum), got %d", reduction);
  if (lse_rows != CCE_LSE_ALL_ROWS && lse_rows != CCE_LSE_LABELLED_ROWS)
    return fail(CCE_ERR_INVALID_ARG, "lse_rows must be CCE_LSE_ALL_ROWS or CCE_LSE_LABELLED_ROWS, got %d", lse_rows);
  *bytes = fwd_layout(nullptr, N, d, V, reduction, lse_rows).bytes;
  return CCE_OK;
}

int cce_backward_workspace_bytes(int64_t N, int64_t d, int64_t V, int64_t chunk_size, int need_grad_hidden,
                                 int grad_hidden_dtype, int need_grad_weight, int grad_weight_dtype, size_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return fail(CCE_ERR_INVALID_ARG, "bytes must not be null");
  int rc = check_dims(N, d, V);
  if (rc) return rc;
  if ((need_grad_hidden && grad_hidden_dtype != CCE_DTYPE_BF16 && grad_hidden_dtype != CCE_DTYPE_F32) ||
      (need_grad_weight && grad_weight_dtype != CCE_DTYPE_BF16 && grad_weight_dtype != CCE_DTYPE_F32))
    return fail(CCE_ERR_INVALID_ARG, "gradient dtypes must be CCE_DTYPE_BF16 or CCE_DTYPE_F32");
  *bytes = bwd_layout(nullptr, N, d, V, band_width(V, chunk_size, N, d), need_grad_hidden != 0,
                      need_grad_weight != 0, grad_hidden_dtype == CCE_DTYPE_F32,
                      grad_weight_dtype == CCE_DTYPE_F32).bytes;
  return CCE_OK;
}

int cce_forward(const void* hidden, const void* weight, const void* labels, int labels_int64, const float* bias,
                int64_t N, int64_t d, int64_t V, int64_t ignore_index, float label_smoothing, float z_loss_weight,
                int smoothing_form, int reduction, int lse_rows, float* loss_out, float* lse_out, float* target_out,
                int32_t* n_valid_out, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return forward_run(hidden, weight, labels, labels_int64, bias, N, d, V, ignore_index, label_smoothing,
                     z_loss_weight, smoothing_form, reduction, lse_rows, loss_out, lse_out, target_out, n_valid_out,
                     workspace, workspace_bytes, stream);
}

int cce_forward_noalloc(const void* hidden, const void* weight, const void* labels, int labels_int64,
                        const float* bias, int64_t N, int64_t d, int64_t V, int64_t ignore_index,
                        float label_smoothing, float z_loss_weight, int smoothing_form, int reduction, int lse_rows,
                        float* loss_out, float* lse_out, float* target_out, int32_t* n_valid_out, void* stream) {
  g_err[0] = 0;
  int rc = check_dims(N, d, V);
  if (rc) return rc;
  if (reduction < CCE_REDUCTION_NONE || reduction > CCE_REDUCTION_SUM)
    return fail(CCE_ERR_INVALID_ARG, "reduction must be 0 (none), 1 (mean) or 2 (sum), got %d", reduction);
  if (lse_rows != CCE_LSE_ALL_ROWS && lse_rows != CCE_LSE_LABELLED_ROWS)
    return fail(CCE_ERR_INVALID_ARG, "lse_rows must be CCE_LSE_ALL_ROWS or CCE_LSE_LABELLED_ROWS, got %d", lse_rows);
  // the static scratch is fixed: the rows are read in place wherever the
  // byte offsets into hidden allow, so no N x d copy takes scratch
  const size_t need = fwd_layout(nullptr, N, d, V, reduction, lse_rows, true).bytes;
  if (need > (size_t)CCE_NOALLOC_SCRATCH_BYTES)
    return fail(CCE_ERR_WORKSPACE,
                "cce_forward_noalloc: this problem (N=%ld d=%ld V=%ld) needs %zu bytes of scratch, more than the "
                "%zu-byte static scratch; call cce_forward with a workspace instead",
                (long)N, (long)d, (long)V, need, (size_t)CCE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return forward_run(hidden, weight, labels, labels_int64, bias, N, d, V, ignore_index, label_smoothing,
                     z_loss_weight, smoothing_form, reduction, lse_rows, loss_out, lse_out, target_out, n_valid_out,
                     ws, (size_t)CCE_NOALLOC_SCRATCH_BYTES, stream, true);
}

int cce_backward(const float* grad_out, const void* hidden, const void* weight, const void* labels, int labels_int64,
                 const float* bias, const float* lse, const int32_t* n_valid, int64_t N, int64_t d, int64_t V,
                 int64_t ignore_index, float label_smoothing, float z_loss_weight, int reduction, int64_t chunk_size,
                 void* grad_hidden, int grad_hidden_dtype, void* grad_weight, int grad_weight_dtype,
                 float* grad_bias, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_dims(N, d, V);
  if (rc) return rc;
  if (reduction < CCE_REDUCTION_NONE || reduction > CCE_REDUCTION_SUM)
    return fail(CCE_ERR_INVALID_ARG, "reduction must be 0 (none), 1 (mean) or 2 (sum), got %d", reduction);
  if ((grad_hidden && grad_hidden_dtype != CCE_DTYPE_BF16 && grad_hidden_dtype != CCE_DTYPE_F32) ||
      (grad_weight && grad_weight_dtype != CCE_DTYPE_BF16 && grad_weight_dtype != CCE_DTYPE_F32))
    return fail(CCE_ERR_INVALID_ARG, "gradient dtypes must be CCE_DTYPE_BF16 or CCE_DTYPE_F32");
  if (N > 0 && (!grad_out || !hidden || !weight || !labels || !lse || !n_valid))
    return fail(CCE_ERR_INVALID_ARG, "grad_out, hidden, weight, labels, lse and n_valid must not be null");
  if (!(label_smoothing >= 0.f && label_smoothing <= 1.f))
    return fail(CCE_ERR_INVALID_ARG, "label_smoothing must be in [0, 1]");
  if (misaligned(hidden) || misaligned(weight) || misaligned(workspace) || misaligned(grad_hidden) ||
      misaligned(grad_weight))
    return fail(CCE_ERR_INVALID_ARG, "hidden, weight, gradients and workspace must be 16-byte aligned");
  const bool need_dh = grad_hidden != nullptr, need_dw = grad_weight != nullptr, need_db = grad_bias != nullptr;
  if (need_db && !bias) return fail(CCE_ERR_INVALID_ARG, "grad_bias requested without bias");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool dh_f32 = grad_hidden_dtype == CCE_DTYPE_F32, dw_f32 = grad_weight_dtype == CCE_DTYPE_F32;
  const long Vb = band_width(V, chunk_size, N, d);
  const BwdLayout need = bwd_layout(nullptr, N, d, V, Vb, need_dh, need_dw, dh_f32, dw_f32);
  if (workspace_bytes < need.bytes || (need.bytes && !workspace))
    return fail(CCE_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need.bytes, workspace_bytes);
  if (N == 0) {
    if (need_dw) {
      rc = zero_fill(grad_weight, (size_t)V * d * (dw_f32 ? 4 : 2), st);
      if (rc) return rc;
    }
    if (need_db) return zero_fill(grad_bias, (size_t)V * 4, st);
    return CCE_OK;
  }
  if (!need_dh && !need_dw && !need_db) return CCE_OK;
  BwdLayout L = bwd_layout(workspace, N, d, V, Vb, need_dh, need_dw, dh_f32, dw_f32);
  if (L.ht_out) L.HT = static_cast<bf16_t*>(grad_hidden);
  if (L.wt_dh) {
    L.WT[0] = static_cast<bf16_t*>(grad_hidden);
    L.WT[1] = L.WT[0] + d * Vb;
  }
  const long NT = ht_cols(N);  // row length of H^T
  const bf16_t* H = static_cast<const bf16_t*>(hidden);
  const bf16_t* W = static_cast<const bf16_t*>(weight);

  // Banded backward: the rows with a label are compacted to the front (the
  // GEMMs then skip the row tiles past them); the rest of dH is zeroed here.
  if (L.idx) {
    hipLaunchKernelGGL(compact_rows_kernel, dim3(1), dim3(1024), 0, st, labels, labels_int64, (int)N,
                       (long)ignore_index, L.idx, L.live, 0, 0, 0);
    HIP_TRY(hipGetLastError());
    if (L.Hc) {
      const long chunks = (long)N * (d / 8);
      hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)std::min<long>(ceil_div(chunks, 256), 8192)), dim3(256),
                         0, st, H, (int)d, L.idx, (int)N, L.Hc);
      HIP_TRY(hipGetLastError());
    }
  }
  hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)ceil_div(N, 256)), dim3(256), 0, st, grad_out, lse, n_valid,
                     labels, labels_int64, (int)N, (int)V, (long)ignore_index, label_smoothing, z_loss_weight,
                     reduction, L.idx, L.rowp, L.rowlab);
  HIP_TRY(hipGetLastError());
  if (need_dw) {
    hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)ceil_div(NT, 64), (unsigned)ceil_div(d, 64)), dim3(256), 0,
                       st, L.Hc ? L.Hc : H, (long)d, (int)N, (int)d, L.HT, (long)NT, (int)NT,
                       L.Hc ? nullptr : L.idx);
    HIP_TRY(hipGetLastError());
  }

  // Work units (b, r): vocabulary band b, row block r (rows [r*Nb, r*Nb +
  // Nb) of the compacted order), band-major.  Each unit's gradient block G
  // (rows x band) lives in G[u & 1] for unit u = b * nblocks + r.
  const long nbands = ceil_div(V, Vb);
  const int R = L.nblocks;
  const long Nb = L.Nb;
  const long units = nbands * R;
  // The partial band (V - (nbands - 1) * Vb columns) comes first: its logits
  // recompute then runs alone, where it is shortest, and the last launch,
  // which has no next unit's recompute to fill the CUs its long dW tiles
  // leave idle, gets a full band.
  const long head = V - (nbands - 1) * Vb;
  auto band_cols = [&](long b, long& v0, long& vb, long& vb64) {
    v0 = b == 0 ? 0 : head + (b - 1) * Vb;
    vb = b == 0 ? head : Vb;
    vb64 = (long)align_up((size_t)vb, 64);
  };
  auto block_span = [&](long r, long& m0, long& rows) {
    m0 = r * Nb;
    rows = std::min<long>(Nb, N - m0);
  };
  // dH accumulates over the bands: the first band stores, middle bands add,
  // the last writes the output (fp32 dH: the output is the accumulator; with
  // grad_hidden holding H^T or W^T the last band adds too, and dH is written
  // afterwards)
  auto dh_mode = [&](long b) {
    if (nbands == 1) return 0;
    if (dh_f32) return b == 0 ? 0 : 4;
    return b == 0 ? 1 : (b == nbands - 1 && !L.dh_late ? 3 : 2);
  };
  // dW of a band accumulates over the row blocks in the same way (the last
  // band's W^T in its own rows of grad_weight: written afterwards)
  auto dw_mode = [&](long b, long r) {
    if (R == 1) return 0;
    if (dw_f32) return r == 0 ? 0 : 4;
    return r == 0 ? 1 : (r == R - 1 && !(L.wt_last_in_place && b == nbands - 1) ? 3 : 2);
  };
  // rows [v0, v0 + vb) of grad_weight, as bf16 elements
  auto dw_rows = [&](long b) {
    const long v0 = b == 0 ? 0 : head + (b - 1) * Vb;
    return reinterpret_cast<bf16_t*>(static_cast<char*>(grad_weight) + v0 * d * (dw_f32 ? 4 : 2));
  };
  // where W^T of band b lives ([d][Vb], see BwdLayout::wt_out)
  auto wt_of = [&](long b) -> bf16_t* {
    if (!L.wt_out) return L.WT[b & 1];
    if (b + 1 < nbands) return dw_rows(b + 1);
    return L.wt_last_in_place ? dw_rows(b) : L.WT[0];
  };
  // dH of unit (b, r): G[rows][vb64] . WT[d][vb64]^T over hidden columns [c0, c0 + nc)
  auto dh_shape = [&](long b, long r, const bf16_t* G, long c0, long nc, GemmShape& g, AccParams& e) {
    long v0, vb, vb64, m0, rows;
    band_cols(b, v0, vb, vb64);
    block_span(r, m0, rows);
    g.A = G; g.lda = Vb; g.B = wt_of(b) + c0 * Vb; g.ldb = Vb;
    g.M = (int)rows; g.N = (int)nc; g.K = (int)vb64;
    g.live = L.live; g.dyn = L.live ? kDynM : kDynNone; g.live_base = (int)m0;
    e.rowmap = L.idx ? L.idx + m0 : nullptr;
    e.acc32 = L.dHacc ? L.dHacc + m0 * d + c0 : nullptr; e.ldacc = d;
    // with a row map the output rows are global (the map holds them);
    // without one (no compaction) the block's rows start at m0
    const long orow = L.idx ? 0 : m0;
    e.out = dh_f32 ? static_cast<void*>(static_cast<float*>(grad_hidden) + orow * d + c0)
                   : static_cast<void*>(static_cast<bf16_t*>(grad_hidden) + orow * d + c0);
    e.ldo = d;
    e.out_f32 = dh_f32;
    e.mode = dh_mode(b);
  };
  // dW of unit (b, r): rows [v0, v0 + vb), hidden columns [c0, c0 + nc) of
  // grad_weight = G^T . H over the block's rows
  auto dw_shape = [&](long b, long r, const bf16_t* G, long c0, long nc, GemmShape& g, AccParams& e) {
    long v0, vb, vb64, m0, rows;
    band_cols(b, v0, vb, vb64);
    block_span(r, m0, rows);
    g.A = G; g.lda = Vb;  // MN-major: element (v, n) at G[n*Vb + v]
    g.B = L.HT + c0 * NT; g.ldb = NT; g.kb = (int)m0;  // H^T columns [m0, m0 + rows)
    g.M = (int)vb; g.N = (int)nc; g.K = (int)rows;
    g.live = L.live; g.dyn = L.live ? kDynK : kDynNone; g.live_base = (int)m0;
    e.rowmap = nullptr;
    e.acc32 = L.dWacc ? L.dWacc + c0 : nullptr; e.ldacc = d;
    const long o = v0 * d + c0;
    e.out = dw_f32 ? static_cast<void*>(static_cast<float*>(grad_weight) + o)
                   : static_cast<void*>(static_cast<bf16_t*>(grad_weight) + o);
    e.ldo = d;
    e.out_f32 = dw_f32;
    e.mode = dw_mode(b, r);
  };
  // WT[b & 1][j][c] = W[v0 + c][j], zero for vb <= c < vb64: as its own
  // launch, or as the transpose population of an earlier launch
  auto transpose_params = [&](long b, TransposeParams& t) -> int {
    long v0, vb, vb64;
    band_cols(b, v0, vb, vb64);
    t.in = W + v0 * d; t.ldi = d; t.R = (int)vb; t.C = (int)d;
    t.out = wt_of(b); t.ldo = Vb; t.Rpad = (int)vb64;
    t.tiles_r = (int)ceil_div(vb64, 64);
    return t.tiles_r * (int)ceil_div(d, 64);
  };
  auto transpose_band = [&](long b) -> int {
    TransposeParams t;
    const int tiles = transpose_params(b, t);
    hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)t.tiles_r, (unsigned)(tiles / t.tiles_r)), dim3(256), 0, st,
                       t.in, t.ldi, t.R, t.C, t.out, t.ldo, t.Rpad, nullptr);
    HIP_TRY(hipGetLastError());
    return CCE_OK;
  };
  // dB[v0 .. v0 + vb) = sum over the block's rows of G, added over the blocks
  auto colsum_unit = [&](long b, long r, const bf16_t* G) -> int {
    long v0, vb, vb64, m0, rows;
    band_cols(b, v0, vb, vb64);
    block_span(r, m0, rows);
    hipLaunchKernelGGL(colsum_kernel, dim3((unsigned)ceil_div(vb, 64)), dim3(256), 0, st, G, (long)Vb, (int)rows,
                       (int)vb, L.live, (int)m0, r > 0 ? 1 : 0, grad_bias + v0);
    HIP_TRY(hipGetLastError());
    return CCE_OK;
  };
  auto grad_unit = [&](long u, bool in_band, int bn, GemmShape& g, GradParams& e, int& nb) {
    long v0, vb, vb64, m0, rows;
    band_cols(u / R, v0, vb, vb64);
    block_span(u % R, m0, rows);
    grad_shape(H, W, bias, L, L.G[u & 1], m0, rows, d, v0, vb, bn, in_band, g, e, nb);
  };

  if (banded(d)) {
    // launch u: dW and dH of unit u from G[u & 1] and the recompute of unit
    // u+1 into G[(u+1) & 1]; unit 0's recompute runs alone first.
    const long dmain = band_dmain(d);
    {
      GemmShape g1 = {};
      GradParams e1 = {};
      int nb1 = 0;
      grad_unit(0, false, kFastBN, g1, e1, nb1);
      if (g1.arow) {
        // reading H through the row order: run it as a band launch with only
        // this recompute population (the stand-alone GEMM kernel with the row
        // map spills registers; the band kernel's allocation does not)
        BandLaunch p0 = {};
        p0.gr = g1;
        p0.e_gr = e1;
        p0.nb_gr = nb1;
        rc = launch_band(p0, bias != nullptr, st, CCE_KERNEL_BWD_GRAD);
      } else
        rc = bias ? launch_gemm<kFastBN, kWarp8, true, true, EpiGradBias, 4>(g1, e1, nb1, st, CCE_KERNEL_BWD_GRAD,
                                                                              false)
                  : launch_gemm<kFastBN, kWarp8, true, true, EpiGrad, 4>(g1, e1, nb1, st, CCE_KERNEL_BWD_GRAD, false);
      if (rc) return rc;
      if (need_dh) {
        rc = transpose_band(0);
        if (rc) return rc;
      }
    }
    // With 4 or more splits (very few rows) the band launches are short and the
    // reduction rides in the next launch, so the partials alternate between
    // two buffers; with 2-3 splits the launches are full and it runs as a
    // launch of its own after each unit, on the one buffer.
    const bool fold = L.dhpart && dh_fold(L.dh_ks);
    auto dh_part = [&](long u) { return L.dhpart + (fold ? (u & 1) : 0) * (long)L.dh_ks * Nb * d; };
    // the reduction of unit u's K-split dH partials, with its band's
    // accumulator mode (as dh_shape sets it)
    auto dh_reduction = [&](long u, int ks) {
      const long b = u / R;
      long m0, rows;
      block_span(u % R, m0, rows);
      DhReduce r;
      r.P = dh_part(u);
      r.stride = Nb * d;
      r.ks = ks; r.N = (int)rows; r.d = (int)d;
      r.live = L.live; r.live_base = (int)m0;
      r.acc = L.dHacc ? L.dHacc + m0 * d : nullptr;
      r.mode = dh_mode(b);
      r.out = L.idx ? grad_hidden
                    : (dh_f32 ? static_cast<void*>(static_cast<float*>(grad_hidden) + m0 * d)
                              : static_cast<void*>(static_cast<bf16_t*>(grad_hidden) + m0 * d));
      r.out_f32 = dh_f32;
      r.rowmap = L.idx ? L.idx + m0 : nullptr;
      return r;
    };
    int prev_ks = 1;
    for (long u = 0; u < units; ++u) {
      const long b = u / R, r = u % R;
      const bf16_t* G = L.G[u & 1];
      BandLaunch p = {};
      if (need_dw) {
        if (dmain > 0) {
          dw_shape(b, r, G, 0, dmain, p.dw, p.e_dw);
          p.nb_dw = (int)(ceil_div(p.dw.M, kBM) * ceil_div(dmain, kFastBN));
        }
        if (dmain < d) {
          dw_shape(b, r, G, dmain, d - dmain, p.dw2, p.e_dw2);
          p.nb_dw2 = (int)(ceil_div(p.dw2.M, kBM) * ceil_div(d - dmain, kSlowBN));
        }
      }
      if (need_dh) {
        // the next band's W rows, transposed into the other WT buffer by the
        // band's first launch (band b reads WT[b & 1] in all its launches);
        // the last band's W^T, when it takes the memory that this band's
        // W^T occupies (wt_last_in_place), by a launch of its own once this
        // band is done
        const bool tr_late = L.wt_last_in_place && b + 2 == nbands;
        if (r == 0 && b + 1 < nbands && !tr_late) p.nb_tr = transpose_params(b + 1, p.tr);
        long m0, rows;
        block_span(r, m0, rows);
        const int gm = (int)ceil_div(rows, kBM);
        // K splits of this unit: every split non-empty and a whole number of slabs
        int ks = 1;
        if (L.dhpart) {
          long v0, vb, vb64;
          band_cols(b, v0, vb, vb64);
          p.dh_kc = (int)align_up((size_t)ceil_div(vb64, L.dh_ks), 64);
          ks = (int)ceil_div(vb64, p.dh_kc);
        }
        p.dh_split = L.dhpart != nullptr;  // every unit, even one left with a single split
        p.dh_ks = ks;
        p.dh_part_stride = Nb * d;
        float* const part = L.dhpart ? dh_part(u) : nullptr;
        if (dmain > 0) {
          dh_shape(b, r, G, 0, dmain, p.dh, p.e_dh);
          p.nb_dh = gm * (int)ceil_div(dmain, kFastBN) * ks;
          p.e_dh_part = p.e_dh;
          p.e_dh_part.acc32 = part; p.e_dh_part.ldacc = d; p.e_dh_part.mode = 1; p.e_dh_part.rowmap = nullptr;
        }
        if (dmain < d) {
          dh_shape(b, r, G, dmain, d - dmain, p.dh2, p.e_dh2);
          p.nb_dh2 = gm * (int)ceil_div(d - dmain, kSlowBN) * ks;
          p.e_dh2_part = p.e_dh2;
          p.e_dh2_part.acc32 = part ? part + dmain : nullptr; p.e_dh2_part.ldacc = d;
          p.e_dh2_part.mode = 1; p.e_dh2_part.rowmap = nullptr;
        }
        // the previous unit's partials (the other buffer) into the accumulator
        if (fold && u > 0) {
          p.red = dh_reduction(u - 1, prev_ks);
          long pm0, prows;
          block_span((u - 1) % R, pm0, prows);
          p.nb_red = (int)std::min<long>(ceil_div(prows * (d / 4), kWarp8 * 64 * 4), 1024);
        }
        prev_ks = ks;
      }
      if (u + 1 < units) grad_unit(u + 1, true, kFastBN, p.gr, p.e_gr, p.nb_gr);
      rc = launch_band(p, bias != nullptr, st);
      if (rc) return rc;
      if (need_dh && L.dhpart && (!fold || u + 1 == units)) {
        // this unit's partials (the last band's go to the output: mode 0, 3 or 4)
        long m0, rows;
        block_span(r, m0, rows);
        hipLaunchKernelGGL(dh_reduce_kernel, dim3((unsigned)std::min<long>(ceil_div(rows * (d / 4), 256), 2048)),
                           dim3(256), 0, st, dh_reduction(u, prev_ks));
        HIP_TRY(hipGetLastError());
      }
      if (need_dh && L.wt_last_in_place && b + 2 == nbands && r == R - 1) {
        rc = transpose_band(b + 1);
        if (rc) return rc;
      }
      if (need_db) {
        rc = colsum_unit(b, r, G);
        if (rc) return rc;
      }
    }
    // outputs whose memory held W^T / H^T during the bands: the last band's
    // dW from its fp32 accumulator, then dH (the labelled rows) through the
    // row map; the rows without a label are zeroed last
    auto convert = [&](const float* src, long rows, const int* live, const int* rowmap, void* out) {
      DhReduce c = {};
      c.P = src;
      c.ks = 1;
      c.N = (int)rows; c.d = (int)d;
      c.live = live; c.live_base = 0;
      c.mode = 0;
      c.out = out; c.out_f32 = 0;
      c.rowmap = rowmap;
      hipLaunchKernelGGL(dh_reduce_kernel, dim3((unsigned)std::min<long>(ceil_div(rows * (d / 4), 256), 2048)),
                         dim3(256), 0, st, c);
      return hipGetLastError();
    };
    if (L.wt_last_in_place) {
      long v0, vb, vb64;
      band_cols(nbands - 1, v0, vb, vb64);
      HIP_TRY(convert(L.dWacc, vb, nullptr, nullptr, dw_rows(nbands - 1)));
    }
    if (L.dh_late) HIP_TRY(convert(L.dHacc, N, L.live, L.idx, grad_hidden));
    if (need_dh) {
      const long row_bytes = d * (dh_f32 ? 4 : 2);
      hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)std::min<long>(ceil_div(N * (row_bytes / 16), 256), 4096)),
                         dim3(256), 0, st, static_cast<char*>(grad_hidden), row_bytes, L.idx, L.live, (int)N);
      HIP_TRY(hipGetLastError());
    }
    return CCE_OK;
  }

  // d not a multiple of 64: one G buffer; per unit the recompute (register-
  // staged pipeline), then dH and dW
  for (long u = 0; u < units; ++u) {
    const long b = u / R, r = u % R;
    GemmShape g1 = {};
    GradParams e1 = {};
    int nb1 = 0;
    {
      long v0, vb, vb64, m0, rows;
      band_cols(b, v0, vb, vb64);
      block_span(r, m0, rows);
      grad_shape(H, W, bias, L, L.G[0], m0, rows, d, v0, vb, kSlowBN, false, g1, e1, nb1);
    }
    rc = bias ? launch_gemm<kSlowBN, kWarp8, true, true, EpiGradBias, 3>(g1, e1, nb1, st, CCE_KERNEL_BWD_GRAD, false)
              : launch_gemm<kSlowBN, kWarp8, true, true, EpiGrad, 3>(g1, e1, nb1, st, CCE_KERNEL_BWD_GRAD, false);
    if (rc) return rc;
    GemmShape g2 = {}, g3 = {};
    AccParams e2 = {}, e3 = {};
    if (need_dh) {
      if (r == 0) {
        rc = transpose_band(b);
        if (rc) return rc;
      }
      dh_shape(b, r, L.G[0], 0, d, g2, e2);
    }
    if (need_dw) dw_shape(b, r, L.G[0], 0, d, g3, e3);
    if (need_dh && need_dw)
      rc = launch_dual_acc(g3, e3, g2, e2, st);
    else if (need_dh)
      rc = launch_acc<kFastBN, true, 4>(g2, e2, st, CCE_KERNEL_BWD_DH);
    else if (need_dw)
      rc = launch_acc<kSlowBN, false, 5>(g3, e3, st, CCE_KERNEL_BWD_DW);
    if (rc) return rc;
    if (need_db) {
      rc = colsum_unit(b, r, L.G[0]);
      if (rc) return rc;
    }
  }
  return CCE_OK;
}

int cce_logits_forward_workspace_bytes(int64_t N, int64_t V, int reduction, size_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return fail(CCE_ERR_INVALID_ARG, "bytes must not be null");
  const int rc = check_logits_args(N, V, CCE_DTYPE_F32, V, reduction, 0.f, CCE_SMOOTH_LOGV);
  if (rc) return rc;
  *bytes = logits_layout(nullptr, N).bytes;
  return CCE_OK;
}

int cce_logits_forward(const void* logits, int logits_dtype, int64_t ld, const void* labels, int labels_int64,
                       int64_t N, int64_t V, int64_t ignore_index, float label_smoothing, float z_loss_weight,
                       int smoothing_form, int reduction, float* loss_out, float* lse_out, int32_t* n_valid_out,
                       void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_logits_args(N, V, logits_dtype, ld, reduction, label_smoothing, smoothing_form);
  if (rc) return rc;
  // loss_out is [N] for 'none', so it may be null when N == 0
  if (!n_valid_out || (!loss_out && (N > 0 || reduction != CCE_REDUCTION_NONE)) ||
      (N > 0 && (!logits || !labels || !lse_out)))
    return fail(CCE_ERR_INVALID_ARG, "logits, labels, loss_out, lse_out and n_valid_out must not be null");
  const LogitsLayout need = logits_layout(nullptr, N);
  if (workspace_bytes < need.bytes || !workspace)
    return fail(CCE_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need.bytes, workspace_bytes);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const LogitsLayout L = logits_layout(workspace, N);
  float* rowloss = reduction == CCE_REDUCTION_NONE ? loss_out : L.rowloss;
  const float logV = logf((float)V);
  if (N > 0) {
    hipEvent_t e0, e1;
    const bool timed = timing_begin(st, &e0, &e1);
#define CCE_LAUNCH_LFWD(T)                                                                                        \
  hipLaunchKernelGGL(ce_logits_fwd_kernel<T>, dim3((unsigned)N), dim3(256), 0, st, static_cast<const T*>(logits), \
                     (long)ld, labels, labels_int64, (int)V, (long)ignore_index, label_smoothing, z_loss_weight,   \
                     logV, smoothing_form, lse_out, rowloss, L.bsum, L.bcnt)
    if (logits_dtype == CCE_DTYPE_BF16)
      CCE_LAUNCH_LFWD(uint16_t);
    else if (logits_dtype == CCE_DTYPE_F16)
      CCE_LAUNCH_LFWD(_Float16);
    else
      CCE_LAUNCH_LFWD(float);
#undef CCE_LAUNCH_LFWD
    const hipError_t le = hipGetLastError();
    if (timed) {
      const double bytes = (double)N * (double)V * (double)logits_elem_size(logits_dtype);
      timing_end(CCE_KERNEL_LOGITS_FWD, st, e0, e1, bytes, bytes);
    }
    HIP_TRY(le);
  }
  hipLaunchKernelGGL(fwd_finalize_kernel, dim3(1), dim3(1024), 0, st, L.bsum, L.bcnt, (int)N, reduction, loss_out,
                     n_valid_out);
  HIP_TRY(hipGetLastError());
  return CCE_OK;
}

int cce_logits_backward(const float* grad_out, const void* logits, int logits_dtype, int64_t ld, const void* labels,
                        int labels_int64, const float* lse, const int32_t* n_valid, int64_t N, int64_t V,
                        int64_t ignore_index, float label_smoothing, float z_loss_weight, int smoothing_form,
                        int reduction, void* grad_logits, int grad_dtype, int64_t ld_grad, void* stream) {
  g_err[0] = 0;
  int rc = check_logits_args(N, V, logits_dtype, ld, reduction, label_smoothing, smoothing_form);
  if (rc) return rc;
  if (grad_dtype != logits_dtype && grad_dtype != CCE_DTYPE_F32)
    return fail(CCE_ERR_INVALID_ARG, "grad_dtype must be the logits' dtype or CCE_DTYPE_F32, got %d", grad_dtype);
  if (ld_grad < V) return fail(CCE_ERR_INVALID_ARG, "gradient row stride %ld is smaller than V = %ld", (long)ld_grad, (long)V);
  if (grad_logits == logits && (grad_dtype != logits_dtype || ld_grad != ld))
    return fail(CCE_ERR_INVALID_ARG, "grad_logits may alias the logits only with the same dtype and row stride");
  if (N == 0) return CCE_OK;
  if (!grad_out || !logits || !labels || !lse || !n_valid || !grad_logits)
    return fail(CCE_ERR_INVALID_ARG, "grad_out, logits, labels, lse, n_valid and grad_logits must not be null");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipEvent_t e0, e1;
  const bool timed = timing_begin(st, &e0, &e1);
#define CCE_LAUNCH_LBWD(T, TO)                                                                                       \
  hipLaunchKernelGGL((ce_logits_bwd_kernel<T, TO>), dim3((unsigned)N), dim3(256), 0, st, grad_out,                   \
                     static_cast<const T*>(logits), (long)ld, labels, labels_int64, lse, n_valid, (int)V,             \
                     (long)ignore_index, label_smoothing, z_loss_weight, smoothing_form, reduction,                 \
                     static_cast<TO*>(grad_logits), (long)ld_grad)
  const bool f32_out = grad_dtype == CCE_DTYPE_F32;
  if (logits_dtype == CCE_DTYPE_BF16) {
    if (f32_out)
      CCE_LAUNCH_LBWD(uint16_t, float);
    else
      CCE_LAUNCH_LBWD(uint16_t, uint16_t);
  } else if (logits_dtype == CCE_DTYPE_F16) {
    if (f32_out)
      CCE_LAUNCH_LBWD(_Float16, float);
    else
      CCE_LAUNCH_LBWD(_Float16, _Float16);
  } else {
    CCE_LAUNCH_LBWD(float, float);
  }
#undef CCE_LAUNCH_LBWD
  const hipError_t le = hipGetLastError();
  if (timed) {
    const double bytes = (double)N * (double)V * (double)(logits_elem_size(logits_dtype) + logits_elem_size(grad_dtype));
    timing_end(CCE_KERNEL_LOGITS_BWD, st, e0, e1, bytes, bytes);
  }
  HIP_TRY(le);
  return CCE_OK;
}

int cce_logits_forward_backward(const void* logits, int logits_dtype, int64_t ld, const void* labels,
                                int labels_int64, int64_t N, int64_t V, int64_t ignore_index, float label_smoothing,
                                float z_loss_weight, int smoothing_form, int reduction, int grad_mean, float* loss_out,
                                float* lse_out, int32_t* n_valid_out, void* grad_logits, int grad_dtype,
                                int64_t ld_grad, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_logits_args(N, V, logits_dtype, ld, reduction, label_smoothing, smoothing_form);
  if (rc) return rc;
  if (grad_dtype != logits_dtype && grad_dtype != CCE_DTYPE_F32)
    return fail(CCE_ERR_INVALID_ARG, "grad_dtype must be the logits' dtype or CCE_DTYPE_F32, got %d", grad_dtype);
  if (ld_grad < V) return fail(CCE_ERR_INVALID_ARG, "gradient row stride %ld is smaller than V = %ld", (long)ld_grad, (long)V);
  if (grad_logits == logits && (grad_dtype != logits_dtype || ld_grad != ld))
    return fail(CCE_ERR_INVALID_ARG, "grad_logits may alias the logits only with the same dtype and row stride");
  if (!n_valid_out || (!loss_out && (N > 0 || reduction != CCE_REDUCTION_NONE)) ||
      (N > 0 && (!logits || !labels || !lse_out || !grad_logits)))
    return fail(CCE_ERR_INVALID_ARG, "logits, labels, loss_out, lse_out, n_valid_out and grad_logits must not be null");
  const LogitsLayout need = logits_layout(nullptr, N);
  if (workspace_bytes < need.bytes || !workspace)
    return fail(CCE_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need.bytes, workspace_bytes);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const LogitsLayout L = logits_layout(workspace, N);
  float* rowloss = reduction == CCE_REDUCTION_NONE ? loss_out : L.rowloss;
  if (N > 0) {
    if (grad_mean) {
      hipLaunchKernelGGL(count_valid_kernel, dim3(1), dim3(1024), 0, st, labels, labels_int64, (int)N,
                         (long)ignore_index, n_valid_out);
      HIP_TRY(hipGetLastError());
    }
    int dev = 0, cus = 0;
    HIP_TRY(hipGetDevice(&dev));
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // two rows in flight per CU: their first reads are still in the memory-side
    // cache when the second pass re-reads them
    const long rows = (long)(cus > 0 ? cus : 256) * 2;
    const unsigned grid = (unsigned)(N < rows ? N : rows);
    const float logV = logf((float)V);
    const int32_t* nv = grad_mean ? n_valid_out : nullptr;
    hipEvent_t e0, e1;
    const bool timed = timing_begin(st, &e0, &e1);
#define CCE_LAUNCH_LFUSED(T, TO)                                                                                      \
  hipLaunchKernelGGL((ce_logits_fused_kernel<T, TO>), dim3(grid), dim3(kFusedThreads), 0, st,                        \
                     static_cast<const T*>(logits), (long)ld, labels, labels_int64, (int)N, (int)V,                  \
                     (long)ignore_index, label_smoothing, z_loss_weight, logV, smoothing_form, nv, lse_out, rowloss, \
                     L.bsum, L.bcnt, static_cast<TO*>(grad_logits), (long)ld_grad)
    const bool f32_out = grad_dtype == CCE_DTYPE_F32;
    if (logits_dtype == CCE_DTYPE_BF16) {
      if (f32_out)
        CCE_LAUNCH_LFUSED(uint16_t, float);
      else
        CCE_LAUNCH_LFUSED(uint16_t, uint16_t);
    } else if (logits_dtype == CCE_DTYPE_F16) {
      if (f32_out)
        CCE_LAUNCH_LFUSED(_Float16, float);
      else
        CCE_LAUNCH_LFUSED(_Float16, _Float16);
    } else {
      CCE_LAUNCH_LFUSED(float, float);
    }
#undef CCE_LAUNCH_LFUSED
    const hipError_t le = hipGetLastError();
    if (timed) {
      const double bytes =
          (double)N * (double)V * (double)(logits_elem_size(logits_dtype) + logits_elem_size(grad_dtype));
      timing_end(CCE_KERNEL_LOGITS_FUSED, st, e0, e1, bytes, bytes);
    }
    HIP_TRY(le);
  }
  hipLaunchKernelGGL(fwd_finalize_kernel, dim3(1), dim3(1024), 0, st, L.bsum, L.bcnt, (int)N, reduction, loss_out,
                     n_valid_out);
  HIP_TRY(hipGetLastError());
  return CCE_OK;
}

int cce_kernel_timing_enable(int enable) {
  g_err[0] = 0;
  std::lock_guard<std::mutex> lk(g_timing.mu);
  g_timing.enabled = enable != 0;
  return CCE_OK;
}

int cce_kernel_timing_read(int kind, double* total_ms, int64_t* launches, double* credited_flops,
                           double* executed_flops) {
  g_err[0] = 0;
  if (kind < 0 || kind >= CCE_KERNEL_KINDS) return fail(CCE_ERR_INVALID_ARG, "kernel kind %d out of range", kind);
  if (!total_ms || !launches) return fail(CCE_ERR_INVALID_ARG, "total_ms and launches must not be null");
  std::vector<TimedLaunch> recs;
  {
    std::lock_guard<std::mutex> lk(g_timing.mu);
    recs.swap(g_timing.pending[kind]);
  }
  double sum = 0.0, cr = 0.0, ex = 0.0;
  int rc = CCE_OK;
  for (auto& r : recs) {
    float ms = 0.f;
    if (rc == CCE_OK) {
      hipError_t e = hipEventSynchronize(r.ev1);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.ev0, r.ev1);
      if (e != hipSuccess) rc = fail(CCE_ERR_HIP, "kernel timing: %s", hipGetErrorString(e));
    }
    sum += ms;
    cr += r.credited;
    ex += r.executed;
  }
  {
    std::lock_guard<std::mutex> lk(g_timing.mu);
    for (auto& r : recs) {
      g_timing.pool.push_back(r.ev0);
      g_timing.pool.push_back(r.ev1);
    }
  }
  *total_ms = sum;
  *launches = (int64_t)recs.size();
  if (credited_flops) *credited_flops = cr;
  if (executed_flops) *executed_flops = ex;
  return rc;
}

}  // extern "C"
