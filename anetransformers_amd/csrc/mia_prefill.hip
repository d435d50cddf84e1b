// mia_prefill.hip -- the rest of the prefill layer around the attention step
// (mistral/mistral_ane_prefill.h:1081-1110): RMSNorm of the token rows
// (:163-175) and the Q4_0 GEMM on fp32 activations (:999-1042, the reference
// dequantises 128-row tiles to fp32 and calls cblas_sgemm), with epilogues for
// the residual adds and SwiGLU (mistral_model.h:174-199).
//
// GEMM: Y[S][N] = X[S][K] . W[N][K]^T on fp16 MFMA (v_mfma_f32_32x32x16_f16)
// with fp32 accuracy where it matters:
//   - X comes as fp16 hi + lo planes (x = hi + lo to ~2^-22, split by its
//     producer), and both halves go through the MFMA;
//   - W's 4-bit values q - 8 are exact in fp16; the fp16 block scale d is
//     applied in fp32 once per 32-value block: acc += d * (X . q) for the
//     block's partial product, which is what dequantising to fp32 computes.
// Workgroup: 256 threads, 64 tokens x 256 weight rows, 4 waves of 64 x 64;
// each iteration covers 64 K values (two Q4_0 blocks, 36 bytes of each row,
// 4-byte aligned because the blocks per row are even), staged three
// iterations ahead by direct-to-LDS loads (q4_gemm_wide_kernel below).
// The weights are read either in the GGUF layout (rows of blocks) or in the
// GEMM tile layout of q4_pack_kernel (the same bytes regrouped once, so that
// a wave's 64 rows x 2 blocks are one contiguous 2,304-byte tile).
#include <algorithm>

#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {
namespace {

constexpr int kGThreads = 256;
constexpr int kBK = 64;           // K values per iteration (two Q4_0 blocks)

__device__ __forceinline__ float f16_bits_f32(unsigned h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

// Two 4-bit values n0, n1 (in bits 0-3 and 16-19 of v) -> fp16 (n0 - 8, n1 - 8):
// 0x6400 | n is the fp16 number 1024 + n, and 1024 + n - 1032 is exact.
__device__ __forceinline__ unsigned nib2_to_h2(unsigned v) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 x = __builtin_bit_cast(h2, v | 0x64006400u);
  const h2 r = x - (h2){(_Float16)1032.0f, (_Float16)1032.0f};
  return __builtin_bit_cast(unsigned, r);
}

// The epilogue of element (m, n) of the product, v.
template <int MODE>
__device__ __forceinline__ void gemm_epilogue(const GemmParams &p, int m, int n, float v) {
  if (MODE == kGemmStore) {
    if (n < p.rows0)
      p.y0[(size_t)m * p.rows0 + n] = v;
    else if (n < p.rows01)
      p.y1[(size_t)m * (p.rows01 - p.rows0) + (n - p.rows0)] = v;
    else
      p.y2[(size_t)m * (p.N - p.rows01) + (n - p.rows01)] = v;
  } else if (MODE == kGemmAdd) {
    float *y = p.y0 + (size_t)m * p.N + n;
    *y = *y + v;
  } else {  // kGemmSiluMul: y0 holds the gate; gate * sigmoid(gate) * up
#pragma clang fp contract(off)
    float *y = p.y0 + (size_t)m * p.N + n;
    const float g = *y;
    const float sig = 1.0f / (1.0f + expf(-g));
    const float r = (g * sig) * v;
    if (p.ohi != nullptr) {
      const size_t i = (size_t)m * p.N + n;
      const _Float16 h = (_Float16)r;
      p.ohi[i] = h;
      p.olo[i] = (_Float16)(r - (float)h);
    } else {
      *y = r;
    }
  }
}

// ---- the Q4_0 GEMM ----
// Workgroup: 256 threads, 64 tokens x 256 weight rows; wave w owns weight rows
// 64w .. 64w+63 (two 32-row MFMA tiles) against all 64 tokens (two 32-token
// tiles), 32 MFMAs per 64-K iteration.  Everything is staged into LDS by
// direct loads (global_load_lds), kWStages iterations deep, with one
// barrier per iteration:
//   - the activations' hi and lo planes, 64 tokens x 64 K each, shared by the
//     four waves, 16-byte chunk c of token row r at chunk c ^ aswz(r) (any 8
//     consecutive rows of an operand read then cover 128 bytes of banks and
//     any 16 rows 256 bytes);
//   - each wave's own 64 weight rows, 36 bytes (two Q4_0 blocks) each, read
//     back by the wave alone: the B operands are formed from the nibbles in
//     registers (no dequantised tile written to LDS, no row done twice).
// Per 32-value block the MFMA partial products (k-steps 0 and 1, hi then lo
// part of each) are scaled by the block's fp16 scale in fp32:
// acc += d * (X . q), as dequantising the block to fp32 computes.
constexpr int kWN = 256;                          // weight rows per workgroup
constexpr int kWStages = 3;                       // iterations staged ahead
constexpr int kWPlane = 64 * kBK * 2;             // one activation plane: 8 KB
constexpr int kWBRows = 64 * 36;                  // one wave's weight rows: 2304 B
constexpr int kWStage = 2 * kWPlane + 4 * kWBRows;  // 25,600 B

// The GEMM tile layout of a Q4_0 matrix [N][K / 32 blocks], N and K multiples
// of 64: tile (s, i) holds rows 64 s .. 64 s + 63 and blocks 2 i, 2 i + 1 at
// byte (s * (K / 64) + i) * 2304:
//   - bytes h * 1024 + rr * 16 + 8 * bb + j (half h, row rr, block bb, j < 8):
//     byte 8 h + kPackOrder[j] of the block's 16 quant bytes;
//   - bytes 2048 + rr * 4 + 2 * bb: the block's fp16 scale.
// A wave stages its tile with two 16-byte and one 4-byte direct load per
// lane, and a lane (row rr, half h) reads its 16 quant bytes in one 16-byte
// LDS read.  In each 4 bytes the order 0, 2, 1, 3 puts the quant bytes of a
// value pair (2t, 2t + 1) in bytes 0 and 2 (t even) or 1 and 3 (t odd), so a
// shift and a mask give both values' nibbles under the fp16 exponent.
constexpr int kPackTile = 2304;
__device__ constexpr int kPackOrder[8] = {0, 2, 1, 3, 4, 6, 5, 7};

// Chunk swizzle of a 128-byte activation row r: rows r and r + 8 (same bank
// half, same r & 7) get different chunks, so 16 rows read together hit 16
// different 16-byte bank groups, 8 rows 8 different ones.
__device__ __forceinline__ int aswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// 16 (dwordx4) or 4 (dword) bytes per lane from global memory into LDS at
// byte M0 + lane * size; completion is awaited with vmcnt (the compiler does
// not track these loads).
__device__ __forceinline__ void lds_dma16(const void *g, unsigned m) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(m)
      : "memory");
}
__device__ __forceinline__ void lds_dma4(const void *g, unsigned m) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(m)
      : "memory");
}
template <int N>
__device__ __forceinline__ void gemm_wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Tile of workgroup L.  The dispatcher hands workgroup L of a launch to XCD
// L mod 8, and each XCD has its own L2.  Without a K split, weight-row tiles
// run fastest (with 8 | nx every XCD keeps its own row tiles: each weight
// byte is fetched into one L2, the activations into all eight).  With a K
// split, workgroup L takes tile w, XCD g owning the contiguous range of w from
// g * T / 8 (T tiles in all; the first T mod 8 XCDs one more), and w runs over
// the token tiles first, then the weight-row tiles, then the splits: an XCD
// works on whole weight-row tiles of one split, and a token tile's
// activations of a split are fetched by the 8 / splits XCDs of that split
// instead of by all eight (HBM traffic per launch at S 512: W2 302 -> 154 MB,
// Wo 110 -> 60 MB, QKV 110 -> 77 MB; without a split this order fetched ~15 %
// more than the plain one).
__device__ __forceinline__ void gemm_tile_of(int L, int nx, int ny, int nz, int &tx, int &ty,
                                             int &tz) {
  if (nz == 1) {
    tx = L % nx;
    ty = L / nx;
    tz = 0;
    return;
  }
  const int T = nx * ny * nz;
  const int g = L & 7, j = L >> 3;
  const int wi = g * (T >> 3) + min(g, T & 7) + j;
  ty = wi % ny;
  const int r = wi / ny;
  tx = r % nx;
  tz = r / nx;
}

template <int MODE, bool PK>
__global__ __launch_bounds__(kGThreads, 2) void q4_gemm_wide_kernel(GemmParams p) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  int tx, ty, tz;
  gemm_tile_of(blockIdx.x, (p.N + kWN - 1) / kWN, (p.S + 63) / 64, p.ksplit, tx, ty, tz);
  const int n0 = tx * kWN, m0 = ty * 64;
  const int n_all = p.K / kBK;
  const int it0 = (int)((long)n_all * tz / p.ksplit);
  const int n_it = (int)((long)n_all * (tz + 1) / p.ksplit) - it0;
  const int last = it0 + n_it - 1;
  const unsigned sbase = __builtin_amdgcn_readfirstlane((unsigned)(__UINTPTR_TYPE__)smem);

  // Activation loads: wave w fills plane w >> 1, token rows 32 (w & 1) .. +32,
  // four instructions of 8 rows; lane i of instruction j: row
  // r = 32 (w & 1) + 8 j + i / 8, LDS chunk i % 8 = logical chunk (i % 8) ^ aswz(r).
  const _Float16 *asrc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 32 * (w & 1) + 8 * j + (lane >> 3);
    const int c = (lane & 7) ^ aswz(r);
    asrc[j] = ((w >> 1) ? p.alo : p.ahi) + (size_t)min(m0 + r, p.S - 1) * p.K + 8 * c;
  }
  const unsigned a_lds = (unsigned)((w >> 1) * kWPlane + 32 * (w & 1) * (kBK * 2));
  // Weight loads.  GGUF layout: the wave's 64 rows x 9 dwords, nine
  // instructions of 64 dwords; lane i of instruction j: dword q = 64 j + i,
  // row q / 9, dword q % 9.  Tile layout: the wave's tile, two 16-byte loads
  // and one 4-byte load per lane, in order.
  constexpr int kBLoads = PK ? 3 : 9;
  const uint8_t *bsrc[kBLoads];
  if constexpr (PK) {
    // every wave's rows lie in one matrix (its row counts are multiples of
    // 64); a wave past N loads the last tile of rows (its results are not
    // written)
    const int g = min(n0 + 64 * w, p.N - 64);
    const uint8_t *base = g < p.rows0 ? p.w0 : (g < p.rows01 ? p.w1 : p.w2);
    const int lr = g < p.rows0 ? g : (g < p.rows01 ? g - p.rows0 : g - p.rows01);
    const uint8_t *tile = base + (size_t)(lr / 64) * (size_t)(p.K / kBK) * kPackTile;
    bsrc[0] = tile + 16 * lane;
    bsrc[1] = tile + 1024 + 16 * lane;
    bsrc[2] = tile + 2048 + 4 * lane;
  } else {
#pragma unroll
    for (int j = 0; j < kBLoads; ++j) {
      const int q = 64 * j + lane;
      const int g = min(n0 + 64 * w + q / 9, p.N - 1);
      const uint8_t *base = g < p.rows0 ? p.w0 : (g < p.rows01 ? p.w1 : p.w2);
      const int lr = g < p.rows0 ? g : (g < p.rows01 ? g - p.rows0 : g - p.rows01);
      bsrc[j] = base + (size_t)lr * (size_t)(p.K / 32) * 18 + 4 * (q % 9);
    }
  }
  const unsigned b_lds = (unsigned)(2 * kWPlane + w * kWBRows);
  // Iteration `it` (absolute) into stage `st`: 4 + 9 (GGUF) or 4 + 3 (tile)
  // loads per wave.
  auto issue = [&](int st, int it) {
    const unsigned sb = sbase + (unsigned)(st * kWStage);
    // (wave-uniform offsets: one scalar multiply, then a 64-bit add per lane)
    const unsigned aoff = __builtin_amdgcn_readfirstlane((unsigned)it * (unsigned)(kBK * 2));
    const unsigned boff =
        __builtin_amdgcn_readfirstlane((unsigned)it * (PK ? (unsigned)kPackTile : 36u));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      lds_dma16((const char *)asrc[j] + aoff, sb + a_lds + 1024u * j);
    if constexpr (PK) {
      lds_dma16(bsrc[0] + boff, sb + b_lds);
      lds_dma16(bsrc[1] + boff, sb + b_lds + 1024u);
      lds_dma4(bsrc[2] + boff, sb + b_lds + 2048u);
    } else {
#pragma unroll
      for (int j = 0; j < kBLoads; ++j) lds_dma4(bsrc[j] + boff, sb + b_lds + 256u * j);
    }
  };
  constexpr int kLoadsPerStage = 4 + kBLoads;

  f16v acc[2][2];
#pragma unroll
  for (int tm = 0; tm < 2; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[tm][tn][i] = 0.0f;

  typedef __attribute__((address_space(3))) h8 lds_h8;
  typedef __attribute__((address_space(3))) unsigned lds_u32;
  unsigned nib_mask = 0x000F000Fu;  // in a VGPR
  asm volatile("" : "+v"(nib_mask));
  const unsigned nib_exp = __builtin_amdgcn_readfirstlane(0x64006400u);
  auto compute = [&](int st) {
    const unsigned sb = sbase + (unsigned)(st * kWStage);
    // this lane's weight rows (tn): dwords 2h .. 2h+2 (block 0's nibbles
    // 8h .. 8h+7 at byte offset 2), dword 0 (scale 0, low half), dword 4
    // (scale 1, high half), dwords 5+2h, 6+2h (block 1's nibbles 8h .. 8h+7)
    // (tile layout: the lane's 16 quant bytes and the row's two scales)
    unsigned nb[2][2][2];  // [tn][block][dword]: 8 nibble bytes
    float dsc[2][2];       // [tn][block]
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
      unsigned s0, s1;
      if constexpr (PK) {
        typedef __attribute__((address_space(3))) u4 lds_u4;
        const int rr = 32 * tn + col;
        const u4 qv = *(const lds_u4 *)(__UINTPTR_TYPE__)(sb + b_lds +
                                                          (unsigned)(half * 1024 + rr * 16));
        s0 = *(const lds_u32 *)(__UINTPTR_TYPE__)(sb + b_lds + (unsigned)(2048 + rr * 4));
        s1 = s0;
        nb[tn][0][0] = qv[0];
        nb[tn][0][1] = qv[1];
        nb[tn][1][0] = qv[2];
        nb[tn][1][1] = qv[3];
      } else {
        const unsigned rb = sb + b_lds + (unsigned)((32 * tn + col) * 36);
        const lds_u32 *r = (const lds_u32 *)(__UINTPTR_TYPE__)rb;
        const unsigned x0 = r[2 * half], x1 = r[2 * half + 1], x2 = r[2 * half + 2];
        s0 = r[0];
        s1 = r[4];
        nb[tn][0][0] = __builtin_amdgcn_alignbyte(x1, x0, 2);
        nb[tn][0][1] = __builtin_amdgcn_alignbyte(x2, x1, 2);
        nb[tn][1][0] = r[5 + 2 * half];
        nb[tn][1][1] = r[6 + 2 * half];
      }
      dsc[tn][0] = f16_bits_f32(s0);
      dsc[tn][1] = f16_bits_f32(s1 >> 16);
      // converted once here: folded into each FMA, the conversion makes
      // every scale FMA a mixed-precision one
      asm volatile("" : "+v"(dsc[tn][0]), "+v"(dsc[tn][1]));
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      // B operands of the block's two k-steps: values 16 ks + 8h .. +8 are
      // the low (ks 0) or high (ks 1) nibbles of the lane's 8 bytes.  A pair
      // of consecutive bytes goes to the two halves of a dword (GGUF layout:
      // one byte permute; tile layout: a shift, the pair being in bytes 0
      // and 2 or 1 and 3 already), and one AND-OR leaves their nibbles under
      // the fp16 exponent of 1024 (0x6400 | n = 1024 + n); subtracting 1032
      // gives n - 8.
      h8 bop[2][2];  // [ks][tn]
#pragma unroll
      for (int tn = 0; tn < 2; ++tn)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const unsigned x0 = ks && !PK ? nb[tn][kb][0] >> 4 : nb[tn][kb][0];
          const unsigned x1 = ks && !PK ? nb[tn][kb][1] >> 4 : nb[tn][kb][1];
          unsigned v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            unsigned t;
            if constexpr (PK) {
              t = (q < 2 ? x0 : x1) >> (8 * (q & 1) + 4 * ks);
            } else {
              // bytes 2q, 2q+1 of x1:x0 into bytes 0 and 2 (perm selectors
              // 0-3 pick x0's bytes, 4-7 x1's)
              const unsigned sel = (unsigned)(2 * q) | ((unsigned)(2 * q + 1) << 16);
              t = __builtin_amdgcn_perm(x1, x0, sel);
            }
            // (t & mask) | exponent in one instruction (the compiler keeps
            // both constants as literals, which a VOP3 cannot take; one
            // scalar operand at most)
            unsigned e;
            asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(e) : "v"(t), "v"(nib_mask), "s"(nib_exp));
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            v[q] = __builtin_bit_cast(
                unsigned, __builtin_bit_cast(h2, e) - (h2){(_Float16)1032.0f, (_Float16)1032.0f});
          }
          bop[ks][tn] = __builtin_bit_cast(h8, (u4){v[0], v[1], v[2], v[3]});
        }
      f16v blk[2][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int c = 2 * (2 * kb + ks) + half;  // logical 16-byte chunk
        h8 ah[2], al[2];
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
          const int r = 32 * tm + col;
          const unsigned off = (unsigned)(r * (kBK * 2) + 16 * (c ^ aswz(r)));
          ah[tm] = *(const lds_h8 *)(__UINTPTR_TYPE__)(sb + off);
          al[tm] = *(const lds_h8 *)(__UINTPTR_TYPE__)(sb + kWPlane + off);
        }
#pragma unroll
        for (int tm = 0; tm < 2; ++tm)
#pragma unroll
          for (int tn = 0; tn < 2; ++tn) {
            if (ks == 0) {
#pragma unroll
              for (int i = 0; i < 16; ++i) blk[tm][tn][i] = 0.0f;
            }
            blk[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tm], bop[ks][tn], blk[tm][tn], 0, 0, 0);
            blk[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tm], bop[ks][tn], blk[tm][tn], 0, 0, 0);
          }
      }
#pragma unroll
      for (int tn = 0; tn < 2; ++tn)
#pragma unroll
        for (int tm = 0; tm < 2; ++tm)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            acc[tm][tn][i] = __builtin_fmaf(dsc[tn][kb], blk[tm][tn][i], acc[tm][tn][i]);
    }
  };

  // Stage s holds iteration it0 + s (mod kWStages).  Loads past the range
  // repeat its last iteration (in bounds, into a stage nobody reads), so
  // every iteration issues the same number of loads and the waits are exact.
  issue(0, it0);
  issue(1, min(it0 + 1, last));
  auto step = [&](int it, int st) {
    gemm_wait_vmcnt<kLoadsPerStage>();  // this wave's loads of stage st are in
    __syncthreads();                    // everyone's are; stage (it - 1) is read
    issue((st + 2) % kWStages, min(it0 + it + 2, last));
    compute(st);
  };
  int it = 0;
  for (; it + kWStages <= n_it; it += kWStages) {
    step(it, 0);
    step(it + 1, 1);
    step(it + 2, 2);
  }
  if (it < n_it) step(it, 0);
  if (it + 1 < n_it) step(it + 1, 1);
  gemm_wait_vmcnt<0>();  // (the repeated loads past the range)

  // D layout: lane holds column n = col; value i is row 8*(i/4) + 4*half + i%4.
#pragma unroll
  for (int tn = 0; tn < 2; ++tn) {
    const int n = n0 + 64 * w + 32 * tn + col;
    if (n >= p.N) continue;
#pragma unroll
    for (int tm = 0; tm < 2; ++tm) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = m0 + 32 * tm + 8 * (i >> 2) + 4 * half + (i & 3);
        if (m >= p.S) continue;
        if (p.ksplit > 1)
          p.part[((size_t)tz * p.S + m) * p.N + n] = acc[tm][tn][i];
        else
          gemm_epilogue<MODE>(p, m, n, acc[tm][tn][i]);
      }
    }
  }
}

// Sum of the split partial products in split order, then the epilogue.
template <int MODE>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams p) {
  const size_t total = (size_t)p.S * p.N;
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (size_t)gridDim.x * 256) {
    float v = p.part[e];
    for (int z = 1; z < p.ksplit; ++z) v += p.part[(size_t)z * total + e];
    gemm_epilogue<MODE>(p, (int)(e / p.N), (int)(e % p.N), v);
  }
}

// GGUF layout -> GEMM tile layout (above): one thread per (row, block pair),
// 36 bytes in, the same 36 bytes out at their tile places.
__global__ __launch_bounds__(256) void q4_pack_kernel(const uint8_t *__restrict__ src,
                                                      uint8_t *__restrict__ dst, int N, int K) {
  const int steps = K / kBK;
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)N * steps) return;
  const int row = (int)(e / steps), i = (int)(e % steps);
  const unsigned *in = reinterpret_cast<const unsigned *>(src + ((size_t)row * steps + i) * 36);
  unsigned x[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) x[j] = in[j];
  auto byte = [&](int b) { return (x[b >> 2] >> (8 * (b & 3))) & 0xFFu; };
  uint8_t *tile = dst + ((size_t)(row / 64) * steps + i) * kPackTile;
  const int rr = row % 64;
  // block bb: scale at bytes 18 bb, 18 bb + 1; quant bytes at 18 bb + 2 ..
  *reinterpret_cast<unsigned *>(tile + 2048 + 4 * rr) = byte(0) | byte(1) << 8 |
                                                        byte(18) << 16 | byte(19) << 24;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    unsigned o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int bb = d >> 1, j0 = 4 * (d & 1);
      unsigned v = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) v |= byte(18 * bb + 2 + 8 * h + kPackOrder[j0 + j]) << (8 * j);
      o[d] = v;
    }
    *reinterpret_cast<u4 *>(tile + h * 1024 + rr * 16) = (u4){o[0], o[1], o[2], o[3]};
  }
}

// One workgroup per token row: ss = sum(x^2), scale = 1 / sqrt(ss / dim + eps),
// out = (x * scale) * w, the reference's two roundings (vsmul then vmul).
// The GEMM's fp32 activations as fp16 hi + lo planes (x = hi + lo to ~2^-22:
// hi = fp16(x), lo = fp16(x - hi), both rounded to nearest even), split once
// per GEMM input instead of once per column tile of the GEMM.
__global__ __launch_bounds__(256) void split_hilo_kernel(const float *__restrict__ x, long n8,
                                                         _Float16 *__restrict__ hi,
                                                         _Float16 *__restrict__ lo) {
#pragma clang fp contract(off)
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n8; i += (long)gridDim.x * 256) {
    const f4 a = reinterpret_cast<const f4 *>(x)[2 * i];
    const f4 b = reinterpret_cast<const f4 *>(x)[2 * i + 1];
    h8 vh, vl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = e < 4 ? a[e] : b[e - 4];
      const _Float16 h = (_Float16)v;
      vh[e] = h;
      vl[e] = (_Float16)(v - (float)h);
    }
    reinterpret_cast<h8 *>(hi)[i] = vh;
    reinterpret_cast<h8 *>(lo)[i] = vl;
  }
}

// With hi set, the normalised rows go out as the Q4_0 GEMM's fp16 hi + lo
// planes (split exactly as split_hilo_kernel does) instead of fp32 to out.
// 512 threads; thread t sums the 4-value groups at 4t + 2048k in k order, then
// the wave sums and their fixed combination: the order the Q4_0 matvec's
// RMSNorm prologue reproduces.
__global__ __launch_bounds__(512) void rmsnorm_kernel(float *out, const float *in, const float *w,
                                                      int dim, float eps, _Float16 *hi,
                                                      _Float16 *lo) {
#pragma clang fp contract(off)
  __shared__ float red[8];
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *x = in + (size_t)t * dim;
  float ss = 0.0f;
  for (int i = 4 * tid; i < dim; i += 4 * 512) {
    const f4 v = *reinterpret_cast<const f4 *>(x + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
  const size_t row = (size_t)t * dim;
  for (int i = 4 * tid; i < dim; i += 4 * 512) {
    const f4 v = *reinterpret_cast<const f4 *>(x + i);
    const f4 wv = *reinterpret_cast<const f4 *>(w + i);
    f4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (v[e] * scale) * wv[e];
    if (hi != nullptr) {
      h4 vh, vl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 h = (_Float16)r[e];
        vh[e] = h;
        vl[e] = (_Float16)(r[e] - (float)h);
      }
      *reinterpret_cast<h4 *>(hi + row + i) = vh;
      *reinterpret_cast<h4 *>(lo + row + i) = vl;
    } else {
      *reinterpret_cast<f4 *>(out + row + i) = r;
    }
  }
}

template <int MODE>
hipError_t set_wide_lds_limit() {
  const hipError_t e = hipFuncSetAttribute((const void *)q4_gemm_wide_kernel<MODE, false>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           kWStages * kWStage);
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute((const void *)q4_gemm_wide_kernel<MODE, true>,
                             hipFuncAttributeMaxDynamicSharedMemorySize, kWStages * kWStage);
}

template <int MODE>
hipError_t launch_gemm_mode(const GemmParams &p, int num_cus, hipStream_t s, hipEvent_t ev0,
                            hipEvent_t ev1) {
  (void)num_cus;
  const dim3 grid((unsigned)((p.N + kWN - 1) / kWN * ((p.S + 63) / 64) * p.ksplit));
  if (p.packed)
    hipExtLaunchKernelGGL((q4_gemm_wide_kernel<MODE, true>), grid, dim3(kGThreads),
                          kWStages * kWStage, s, ev0, ev1, 0, p);
  else
    hipExtLaunchKernelGGL((q4_gemm_wide_kernel<MODE, false>), grid, dim3(kGThreads),
                          kWStages * kWStage, s, ev0, ev1, 0, p);
  if (p.ksplit > 1) {
    const size_t total = (size_t)p.S * p.N;
    const unsigned blocks = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    hipLaunchKernelGGL(gemm_reduce_kernel<MODE>, dim3(blocks), dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace

long gemm_tiles(int N, int S) { return (long)((N + kWN - 1) / kWN) * ((S + 63) / 64); }

int gemm_pick_ksplit(int N, int K, int S, int num_cus) {
  // Two workgroups fit a CU.  A grid smaller than the CU count splits K
  // (in two or four, keeping at least 8 iterations per split) toward two
  // workgroups per CU; the partial products are summed in split order.
  const long tiles = gemm_tiles(N, S);
  int ks = 1;
  while (ks < 4 && tiles * ks * 2 <= 2L * num_cus && K / kBK / (ks * 2) >= 8) ks *= 2;
  return ks;
}

hipError_t prepare_gemm() {
  const hipError_t e[] = {
      set_wide_lds_limit<kGemmStore>(), set_wide_lds_limit<kGemmAdd>(),
      set_wide_lds_limit<kGemmSiluMul>()};
  for (hipError_t x : e)
    if (x != hipSuccess) return x;
  return hipSuccess;
}

hipError_t launch_q4_gemm(const GemmParams &p, int mode, int num_cus, hipStream_t s,
                          hipEvent_t ev0, hipEvent_t ev1) {
  if (mode == kGemmStore) return launch_gemm_mode<kGemmStore>(p, num_cus, s, ev0, ev1);
  if (mode == kGemmAdd) return launch_gemm_mode<kGemmAdd>(p, num_cus, s, ev0, ev1);
  return launch_gemm_mode<kGemmSiluMul>(p, num_cus, s, ev0, ev1);
}

hipError_t launch_q4_pack(const void *src, void *dst, int N, int K, hipStream_t s) {
  const long n = (long)N * (K / kBK);
  hipLaunchKernelGGL(q4_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     reinterpret_cast<const uint8_t *>(src), reinterpret_cast<uint8_t *>(dst), N,
                     K);
  return hipGetLastError();
}

hipError_t launch_split_hilo(const float *x, long n, _Float16 *hi, _Float16 *lo, int num_cus,
                             hipStream_t s) {
  if (n % 8) return hipErrorInvalidValue;
  const long n8 = n / 8;
  const long wgs = std::min<long>((n8 + 255) / 256, 8L * num_cus);
  hipLaunchKernelGGL(split_hilo_kernel, dim3((unsigned)std::max<long>(wgs, 1)), dim3(256), 0, s,
                     x, n8, hi, lo);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(float *out, const float *in, const float *w, int dim, int S, float eps,
                          hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(S), dim3(512), 0, s, out, in, w, dim, eps,
                     (_Float16 *)nullptr, (_Float16 *)nullptr);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_split(_Float16 *hi, _Float16 *lo, const float *in, const float *w,
                                int dim, int S, float eps, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(S), dim3(512), 0, s, (float *)nullptr, in, w, dim, eps,
                     hi, lo);
  return hipGetLastError();
}

}  // namespace mia
