// mia_flash.hip -- S>1 causal GQA attention on fp16 MFMA for gfx950.
//
// Replaces mistral/mistral_ane_prefill.h:207-275 (attention_batch) and, with
// staged drafts, the sequential verify of mistral/speculative.h:92-101.
//
// Rows are (query t, head g) pairs of one kv head, row = 4t + g, so the four
// query heads of a group share every K/V tile.  A workgroup owns RT = 32*NB
// rows (NB = 2 for prefill: 16 queries x 4 heads) and has four waves, one per
// SIMD.  Every wave works on all RT rows over every fourth 32-key tile of the
// key range (a key group), so K/V tiles are private to a wave: no barrier in
// the tile loop, and each fp16 K/V byte read from LDS feeds 64 rows of MFMA
// work.  The four partial results are merged through LDS at the end.
//
// Per wave and 32-key tile:
//   K, V tiles        global -> LDS directly (global_load_lds, 16 B per lane),
//                     double-buffered, issued one tile ahead of use
//   S^T = K . Q^T     v_mfma_f32_32x32x16_f16, A = K rows (ds_read_b128),
//                     B = Q^T held in registers as two fp16 parts, hi and
//                     lo (q = hi + lo to ~2^-22, RoPE and scale applied):
//                     each k-step is two MFMAs, so the scores carry fp32 q
//                     accuracy (fp16 q alone errs by 2^-12 |q| |k| per
//                     score, visible in the output once scores are large)
//   online softmax    one row per lane (the D column): running max and sum
//                     stay lane-local; the two key halves of a row meet via
//                     a lane exchange; the fp32 exponentials are summed in
//                     fp32 and split into fp16 hi + lo parts for P.V
//                     (p = hi + lo to ~2^-22: a single fp16 P would err by
//                     up to 2^-11 of each weight, 2^-11 |v| in a peaked row)
//   O^T += V^T . P^T  P^T straight from the S^T accumulator layout, hi then
//                     lo part (two MFMAs per k-step), V^T via the
//                     transposing LDS read ds_read_b64_tr_b16
// The scores of tile i+1 are computed on MFMA while the exponentials of tile
// i are formed.  Each row's softmax reference is fixed for the whole key
// range (its first tile's max, subtracted inside the score MFMA by one extra
// k-step), so the loop neither tracks maxima nor rescales; a row whose later
// scores overflow or underflow the fp16 P shows it in its row sum, and its
// wave runs again from the exact row maxima.
//
// Query t at position start+t attends the window [pos-L+1, pos], L =
// min(pos+1, max_seq) (mistral_ane_prefill.h:220-241); positions >= start come
// from the staging buffer when one is given, which keeps the ring untouched
// until the caller commits (sequential-verify semantics on a wrapped ring).
// With p.rope_cs set, Q is rotated by the adjacent-pair RoPE of
// mistral_model.h:79-122 using the per-position (cos, sin) table the K rotation
// kernel wrote.  Masks are applied only to tiles that cross a window edge.
// Very long key ranges over few rows are also split over workgroups and merged
// by flash_merge_kernel.
#include <climits>
#include <type_traits>

#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

constexpr int kKT = 32;     // keys per tile
constexpr int kWaves = 4;   // key groups per workgroup, one wave each

// K/V/Q tiles live in LDS unpadded, one 256 B row per key (or query row),
// with the 16-byte chunk c of row r stored at chunk c ^ swz(r): 16 rows read
// at the same logical chunk then hit 16 distinct bank groups.
__device__ __forceinline__ int swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

__device__ __forceinline__ int window_lo(int pos, int max_seq) {
  // pos - min(pos+1, M) + 1
  return pos + 1 > max_seq ? pos + 1 - max_seq : 0;
}

typedef short s4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));
// LDS (address space 3) pointers: 32-bit addressing, no generic-pointer checks.
typedef __attribute__((address_space(3))) _Float16 lds_half;
typedef __attribute__((address_space(3))) s4 lds_s4;
typedef __attribute__((address_space(3))) h8 lds_h8;
typedef __attribute__((address_space(3))) u4 lds_u4;
typedef __attribute__((address_space(3))) f4 lds_f4;
typedef __attribute__((address_space(3))) f2 lds_f2;
typedef __attribute__((address_space(3))) float lds_float;

template <int NB>
struct Lay {
  static constexpr int kRows = 32 * NB;
  static constexpr int kTileHalfs = kKT * HD;                  // 8 KB
  static constexpr int kBufBytes = kWaves * 4 * kTileHalfs * 2;  // [wave][K0 K1 V0 V1]
  static constexpr int kQBytes = kRows * HD * 2;               // fp16 Q rows
  static constexpr int kMLBytes = kWaves * kRows * 8;          // (max, sum) per wave, row
  // After its loop a wave's own tile buffers hold its partial output:
  // [NB (block)][4 (dim block)][4 chunks][64 lanes][4 floats].
  // Prologue only: (cos, sin) rows of the wave's queries, 2 NB rows of 512 B.
  static constexpr int kCSBytes = kWaves * 2 * NB * 512;
  static constexpr int kBytes = kBufBytes + kQBytes + kMLBytes + kCSBytes;
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ unsigned lds_addr(lds_half *p) {
  return __builtin_amdgcn_readfirstlane((unsigned)(__UINTPTR_TYPE__)p);
}

// 16 bytes per lane from global memory straight into LDS: lane i's data lands
// at byte 16*i of the 1 KB block at LDS byte address `m` (wave-uniform, taken
// from M0, which is restored afterwards).  Inline assembly, so that the
// compiler neither orders later LDS reads of the other buffer behind it nor
// waits for it; completion is awaited explicitly with vmcnt.  The s_nop covers
// the SALU-writes-M0 -> LDS-DMA wait state.
__device__ __forceinline__ void dma16(const void *g, unsigned m) {
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
// The 8 direct loads of a tile whose 32 rows are consecutive: two groups of
// four, each under one M0 value (the LDS block of its first instruction).
// The immediate offset applies to both the global and the LDS address, so
// instruction jj of a group lands at M0 + 1024 jj and reads base + off[jj] +
// 1024 jj: off[] carries the per-lane row/chunk offset minus 1024 jj.
// base1 is base0 advanced by 16 rows, the second group's M0 is m + 4096.
__device__ __forceinline__ void dma8_sb(const void *base0, const void *base1,
                                        const unsigned (&off)[4], unsigned m) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %5\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %6\n\t"
      "global_load_lds_dwordx4 %2, %6 offset:1024\n\t"
      "global_load_lds_dwordx4 %3, %6 offset:2048\n\t"
      "global_load_lds_dwordx4 %4, %6 offset:3072\n\t"
      "s_add_u32 m0, %5, 0x1000\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %7\n\t"
      "global_load_lds_dwordx4 %2, %7 offset:1024\n\t"
      "global_load_lds_dwordx4 %3, %7 offset:2048\n\t"
      "global_load_lds_dwordx4 %4, %7 offset:3072\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(m), "s"(base0), "s"(base1)
      : "memory");
}

// Issues the 8 direct loads of one tensor (K or V) of the 32-key tile kb..kb+31
// (ring slot of key kb: slot0; key range ending at ke) into the wave's tile
// at LDS byte address dst.
// Instruction j moves keys 4j..4j+3: lane i fetches key 4j + i/16, logical
// chunk (i%16) ^ swz(key), which the hardware writes at byte 16*i of the
// instruction's 1 KB block.  swz(4j + i/16) only depends on j through j mod 4,
// so a tile of 32 consecutive ring slots takes a uniform base (row 0 or 16)
// plus one of four per-lane offsets boff[j % 4] (in the form dma8_sb takes);
// tiles that wrap, end early or reach into the staging buffer take per-lane
// addresses.
__device__ __forceinline__ void load_tile(const _Float16 *ring, const _Float16 *stage, int kb,
                                          int slot0, int ke, int start_pos, int max_seq,
                                          int kv_dim, int kv_off, const unsigned (&boff)[4],
                                          int lane, unsigned dst) {
  const bool contiguous =
      kb + kKT <= ke && slot0 + kKT <= max_seq && (stage == nullptr || kb + kKT <= start_pos);
  if (contiguous) {
    const _Float16 *base = ring + (size_t)slot0 * kv_dim;
    dma8_sb(base, base + (size_t)16 * kv_dim, boff, dst);
    return;
  }
  // kb through readfirstlane: keeps the per-lane keys of this rare path from
  // being strength-reduced into loop-carried registers.
  const int kbu = __builtin_amdgcn_readfirstlane(kb);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = 4 * j + (lane >> 4);
    const int kp = min(kbu + r, ke - 1);
    const _Float16 *src;
    if (stage != nullptr && kp >= start_pos) {
      src = stage + (size_t)(kp - start_pos) * kv_dim;
    } else {
      int slot = slot0 + (kp - kbu);
      slot = max_seq >= kKT ? (slot >= max_seq ? slot - max_seq : slot) : slot % max_seq;
      src = ring + (size_t)slot * kv_dim;
    }
    dma16(src + kv_off + 8 * ((lane & 15) ^ swz(r)), dst + 1024u * j);
  }
}

__device__ __forceinline__ h8 lds_read_h8(unsigned addr) {
  return *(const lds_h8 *)(__UINTPTR_TYPE__)addr;
}
__device__ __forceinline__ h4 lds_read_tr4(unsigned addr) {
  return __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(__UINTPTR_TYPE__)addr));
}

// Operand reads from a swizzled tile.  The swizzle XORs disjoint bit fields
// of the byte address, so every read is a per-lane base XOR a compile-time
// constant (plus an immediate offset), one VALU op instead of a register.
//  K (A operand of S^T = K.Q^T), k-step st: row = col, logical chunk
//    2*st + half -> byte ka_base ^ (st << 5), with
//    ka_base = tile + col*256 + 16*(half ^ bit3(col)) + 32*(col & 7).
//  V^T (A operand of O^T += V^T.P^T), k-step kst, dim block db, key half hi:
//    the transposing read of keys 16*kst + 8*hi + 4*half + (i/4) (i = lane%16)
//    at dims 32*db + 16*bit4(lane) + 4*(i%4) -> byte
//    (va_base ^ (64*db ^ 16*hi)) + 2048*hi + 4096*kst, with
//    va_base = tile + 256*u + 8*(i&1) + 16*((2*bit4(lane) + (i&3)/2) ^ 2u),
//    u = 4*half + i/4.
__device__ __forceinline__ unsigned ka_lane_base(int lane) {
  const int col = lane & 31, half = lane >> 5;
  return (unsigned)(col * 256 + 16 * (half ^ ((col >> 3) & 1)) + 32 * (col & 7));
}
__device__ __forceinline__ unsigned va_lane_base(int lane) {
  const int i = lane & 15, half = lane >> 5, l4 = (lane >> 4) & 1;
  const int u = 4 * half + (i >> 2);
  const int c_lane = 2 * l4 + ((i & 3) >> 1);
  return (unsigned)(256 * u + 8 * (i & 1) + 16 * (c_lane ^ (2 * u)));
}
// V^T operand (8 keys x this lane's dim) for k-step kst and dim block db:
// keys {0-3, 8-11} + 4*half of the step, the S^T accumulator's key order.
template <int KST, int DB>
__device__ __forceinline__ h8 read_va(unsigned va_base) {
  const unsigned b0 = va_base ^ (64u * DB);
  const unsigned b1 = va_base ^ (64u * DB ^ 16u);
  const h4 lo = lds_read_tr4(b0 + 4096u * KST);
  const h4 hi = lds_read_tr4(b1 + 4096u * KST + 2048u);
  return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// O^T += V^T . P^T with the accumulator pinned to AGPRs ("+a"): the 128
// output accumulators of a 64-row wave then stay out of the VGPR file, which
// holds the scores, the Q operands and prefetched LDS operands instead.  The
// leading s_nop covers a VALU write of the P operand just before (the hazard
// recognizer does not look inside inline assembly).
__device__ __forceinline__ void mfma_pv(f16v &acc, const h8 &a, const h8 &b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The same with P^T as two fp16 parts, hi then lo (p = hi + lo to ~2^-22):
// the P.V product then carries the fp32 weights' accuracy, where one fp16 P
// errs by up to 2^-11 of each weight (2^-11 |v| in a peaked row).  The second
// MFMA reads the first one's result as SrcC (the same opcode, exactly
// overlapped): no wait states between them.
__device__ __forceinline__ void mfma_pv2(f16v &acc, const h8 &a, const h8 &bh, const h8 &bl) {
  asm("s_nop 1\n\t"
      "v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n\t"
      "v_mfma_f32_32x32x16_f16 %0, %1, %3, %0"
      : "+a"(acc)
      : "v"(a), "v"(bh), "v"(bl));
}
// fp32 pair -> fp16 hi pair and the fp16 pair of what the hi parts miss.
// x - hi is formed by v_fma_mix_f32 straight from the packed fp16 hi (hi *
// -1 + x, one rounding of an exact difference: the same value as converting
// hi back and subtracting, in one instruction instead of two).
__device__ __forceinline__ void split_pair(float x0, float x1, unsigned &hi, unsigned &lo) {
  const h2 h = __builtin_convertvector((f2){x0, x1}, h2);
  hi = __builtin_bit_cast(unsigned, h);
  float r0, r1;
  asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r0) : "v"(hi), "v"(x0));
  asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r1) : "v"(hi), "v"(x1));
  lo = __builtin_bit_cast(unsigned, __builtin_convertvector((f2){r0, r1}, h2));
}
// S^T += K . Q^T over one k-step, hi part then lo part of Q^T, both read
// from AGPRs.  Q^T is loop-invariant (128 registers at 64 rows): held in
// AGPRs, it leaves the VGPR file to the scores, P, the K / V^T operands and
// the addresses, which otherwise spill into AGPRs and are copied back right
// before their MFMAs (the A/B operands of an MFMA may be AGPRs).  Inline
// assembly, so the hazard recognizer does not see that it writes acc: VALU
// readers of acc come after qk_drain.  An MFMA result read as SrcC by the
// next MFMA (exactly overlapped, the same opcode) needs no wait states.
__device__ __forceinline__ void mfma_qk(f16v &acc, const h8 &k, const h8 &qh, const h8 &ql) {
  asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n\t"
      "v_mfma_f32_32x32x16_f16 %0, %1, %3, %0"
      : "+v"(acc)
      : "v"(k), "a"(qh), "a"(ql));
}
// The same as the first MFMAs after VALU writes of acc or of the Q^T AGPRs
// (zeroed scores, the prologue's AGPR writes): the leading wait states cover
// those writes.
__device__ __forceinline__ void mfma_qk_first(f16v &acc, const h8 &k, const h8 &qh,
                                              const h8 &ql) {
  asm("s_nop 4\n\t"
      "v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n\t"
      "v_mfma_f32_32x32x16_f16 %0, %1, %3, %0"
      : "+v"(acc)
      : "v"(k), "a"(qh), "a"(ql));
}
// Before VALU reads of scores written by mfma_qk: more wait states than an
// 8-pass MFMA's result latency, and a data dependence on every score
// register so that no read is scheduled above it.
template <int NB>
__device__ __forceinline__ void qk_drain(f16v (&s)[NB]) {
  if constexpr (NB == 2)
    asm volatile("s_nop 7\n\ts_nop 7" : "+v"(s[0]), "+v"(s[1]));
  else
    asm volatile("s_nop 7\n\ts_nop 7" : "+v"(s[0]));
}

// acc = 0 through the MFMA itself (0 x 0 + 0), so the accumulators are only
// ever written by AGPR-destination MFMAs.  The leading wait states cover a
// VALU write of z just before (a reload of the zero operand, for instance),
// which the hazard recognizer does not see inside inline assembly.
__device__ __forceinline__ void mfma_zero(f16v &acc, const h8 &z) {
  asm volatile("s_nop 4\n\tv_mfma_f32_32x32x16_f16 %0, %1, %1, 0" : "=a"(acc) : "v"(z));
}
// Before VALU reads of accumulators written by mfma_pv: the MFMA result
// latency (wait states the compiler cannot see), and a data dependence on
// every accumulator so that no read is scheduled above it.
template <int NB>
__device__ __forceinline__ void pv_drain(f16v (&o)[NB][4]) {
#pragma unroll
  for (int b = 0; b < NB; ++b)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(o[b][0]), "+a"(o[b][1]), "+a"(o[b][2]), "+a"(o[b][3]));
}

// The same for both row blocks of a 64-row wave with one set of wait states
// (24, more than an 8-pass MFMA's result latency).
template <int NB>
__device__ __forceinline__ void pv_drain_all(f16v (&o)[NB][4]) {
  if constexpr (NB == 2)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]),
                   "+a"(o[1][1]), "+a"(o[1][2]), "+a"(o[1][3]));
  else
    pv_drain<NB>(o);
}

// Combine the two key halves of a row (lanes l and l^32).  ds_bpermute via
// __shfl_xor: clang folds v_permlane32_swap with identical operands as if
// both results were the input, so that builtin is not used here.
__device__ __forceinline__ float half_swap_max(float m) { return fmaxf(m, __shfl_xor(m, 32)); }
__device__ __forceinline__ float half_swap_sum(float x) { return x + __shfl_xor(x, 32); }

// FAST: every key range starts at key 0 of an unwrapped ring with no staged
// rows and holds at least one whole tile (flash_fast_ok), so every tile's 32
// rows are 32 consecutive ring slots: all loads take the uniform-base form,
// and the last, partial tile of a range is loaded as the 32 keys ending at
// the range end, with the keys before the tile's own start masked.  The
// generic kernel handles wrapped windows, staged rows and short ranges with
// per-lane addresses on the tiles that need them.
template <int NB, bool FAST>
__global__ void __launch_bounds__(256) flash_kernel(FlashParams p) {
  using L = Lay<NB>;
  constexpr int RT = 32 * NB;  // rows per workgroup
  extern __shared__ __attribute__((aligned(16))) char smem[];
  lds_half *lds = (lds_half *)smem;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // key group
  const int half = lane >> 5;
  const int col = lane & 31;
  const int kvh = blockIdx.x % p.n_kv;
  const int rest = blockIdx.x / p.n_kv;
  const int rtile = rest % p.n_rtiles;
  const int split = rest / p.n_rtiles;
  const int kv_dim = p.n_kv * HD;
  const int dim_model = kv_dim * 4;
  const int row0 = rtile * RT;

  // Key range of the workgroup (one split), then of this wave.
  const int tq0 = row0 >> 2;
  const int tq1 = min(tq0 + RT / 4 - 1, p.S - 1);
  const int klo = window_lo(p.start_pos + tq0, p.max_seq);
  const int khi = p.start_pos + tq1;
  const int ks = klo + split * p.split_keys;
  const int ke = min(ks + p.split_keys, khi + 1);
  const int nt = ke > ks ? (ke - ks + kKT - 1) / kKT : 0;
  // Key groups interleaved by tile: wave w takes tiles w, w + 4, w + 8, ...
  // of the range.  The waves then share the masked tiles at the causal edge
  // evenly, and every row tile of a kv head walks the same keys in the same
  // order, so its first tiles (and most later ones) are L2 hits after the
  // first workgroup of the head has fetched them.
  const int g_count = nt > w ? (nt - w + kWaves - 1) / kWaves : 0;
  const int kb0 = ks + kKT * w;
  constexpr int kStride = kKT * kWaves;

  // This lane's row in each 32-row block and its window; block-uniform bounds
  // (keys in [lo_max, hi_min] are inside every row's window of the block).
  int lo_t[NB], hi_t[NB], lo_max[NB], hi_min[NB];
  bool valid[NB], bfull[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int t = (row0 + 32 * b + col) >> 2;
    valid[b] = t < p.S;
    const int pos_t = p.start_pos + (valid[b] ? t : p.S - 1);
    lo_t[b] = window_lo(pos_t, p.max_seq);
    hi_t[b] = pos_t;
    const int ts0 = (row0 + 32 * b) >> 2;
    const int ts1 = (row0 + 32 * b + 31) >> 2;
    bfull[b] = ts1 < p.S;
    lo_max[b] = window_lo(p.start_pos + min(ts1, p.S - 1), p.max_seq);
    hi_min[b] = p.start_pos + ts0;
  }
  // Does the lane's row of block b have a key in this wave's range?
  bool has_keys[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    // first tile of the wave ending at or after the row's first key
    const int k0 = max(lo_t[b], ks), k1 = min(hi_t[b], ke - 1);
    const int ahead = k0 - (kb0 + kKT - 1);
    const int i0 = ahead <= 0 ? 0 : (ahead + kStride - 1) / kStride;
    has_keys[b] = valid[b] && k0 <= k1 && i0 < g_count && kb0 + kStride * i0 <= k1;
  }
  // The row bounds are formed here, before the first loads are issued, and
  // not where they are first used (after the wait for Q): pinned, so that the
  // compiler does not sink them into the critical path.
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    int hk = has_keys[b], vb = valid[b], bf = bfull[b];
    asm volatile("" ::"v"(lo_t[b]), "v"(hi_t[b]), "v"(hk), "v"(vb), "s"(bf), "s"(lo_max[b]),
                 "s"(hi_min[b]));
  }

  // Wave-private tile buffers and this lane's direct-load offsets.
  lds_half *kt[2], *vt[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    kt[s] = lds + (w * 4 + s) * L::kTileHalfs;
    vt[s] = lds + (w * 4 + 2 + s) * L::kTileHalfs;
  }
  const unsigned kt_a[2] = {lds_addr(kt[0]), lds_addr(kt[1])};
  const unsigned vt_a[2] = {lds_addr(vt[0]), lds_addr(vt[1])};
  unsigned boff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * j + (lane >> 4);
    boff[j] = (unsigned)(r * kv_dim + kvh * HD + 8 * ((lane & 15) ^ swz(r))) * 2u - 1024u * j;
  }
  const unsigned ka_b[2] = {kt_a[0] + ka_lane_base(lane), kt_a[1] + ka_lane_base(lane)};
  const unsigned va_b[2] = {vt_a[0] + va_lane_base(lane), vt_a[1] + va_lane_base(lane)};
  const _Float16 *const kc = p.kc, *const vc = p.vc;
  const _Float16 *const kst = p.kstage, *const vst = p.vstage;
  auto tile_slot = [&](int i) { return (kb0 + kStride * i) % p.max_seq; };
  // FAST: first key (= ring slot) of the 32 rows loaded for tile i.
  auto fast_slot = [&](int i) { return min(kb0 + kStride * i, ke - kKT); };
  // Ring slots of the next K and V tiles to load, advanced by one stride per
  // load (no division in the tile loop).
  int kslot = 0, vslot = 0;
  auto advance = [&](int s) {
    s += kStride;
    return s < p.max_seq ? s : (s - p.max_seq < p.max_seq ? s - p.max_seq : s % p.max_seq);
  };
#define MIA_LOAD_FAST(ring, i, dst)                                        \
  do {                                                                     \
    const _Float16 *base_ = (ring) + (size_t)fast_slot(i) * kv_dim;        \
    dma8_sb(base_, base_ + (size_t)16 * kv_dim, boff, dst);                \
  } while (0)
#define MIA_LOAD_K(i, buf)                                                                    \
  do {                                                                                        \
    if constexpr (FAST)                                                                       \
      MIA_LOAD_FAST(kc, i, kt_a[buf]);                                                        \
    else                                                                                      \
      load_tile(kc, kst, kb0 + kStride * (i), tile_slot(i), ke, p.start_pos, p.max_seq,       \
                kv_dim, kvh * HD, boff, lane, kt_a[buf]);                                     \
  } while (0)
#define MIA_LOAD_V(i, buf)                                                                    \
  do {                                                                                        \
    if constexpr (FAST)                                                                       \
      MIA_LOAD_FAST(vc, i, vt_a[buf]);                                                        \
    else                                                                                      \
      load_tile(vc, vst, kb0 + kStride * (i), tile_slot(i), ke, p.start_pos, p.max_seq,       \
                kv_dim, kvh * HD, boff, lane, vt_a[buf]);                                     \
  } while (0)
#define MIA_LOAD_K_NEXT(i, buf)                                                              \
  do {                                                                                       \
    if constexpr (FAST) {                                                                    \
      MIA_LOAD_FAST(kc, i, kt_a[buf]);                                                       \
    } else {                                                                                 \
      load_tile(kc, kst, kb0 + kStride * (i), kslot, ke, p.start_pos, p.max_seq, kv_dim,     \
                kvh * HD, boff, lane, kt_a[buf]);                                            \
      kslot = advance(kslot);                                                                \
    }                                                                                        \
  } while (0)
#define MIA_LOAD_V_NEXT(i, buf)                                                              \
  do {                                                                                       \
    if constexpr (FAST) {                                                                    \
      MIA_LOAD_FAST(vc, i, vt_a[buf]);                                                       \
    } else {                                                                                 \
      load_tile(vc, vst, kb0 + kStride * (i), vslot, ke, p.start_pos, p.max_seq, kv_dim,     \
                kvh * HD, boff, lane, vt_a[buf]);                                            \
      vslot = advance(vslot);                                                                \
    }                                                                                        \
  } while (0)
  // K0, K1, then V0: V(i) is first needed one step after K(i+1).
  auto issue_first_tiles = [&]() {
    if (g_count > 0) MIA_LOAD_K(0, 0);
    if (g_count > 1) MIA_LOAD_K(1, 1);
    if (g_count > 0) MIA_LOAD_V(0, 0);
    if constexpr (!FAST) {
      kslot = tile_slot(2);
      vslot = tile_slot(1);
    }
  };
  // Q rows -> fp16 in LDS: RoPE (table of fl32(theta_inv[i] * pos) cos/sin
  // written by the K rotation, mistral_model.h:87-105) and the score scale
  // folded in; rows past the last query are zero.  Each wave stages its own
  // 8 NB rows (queries 2 NB w ..) as fp32, and their (cos, sin) rows, with
  // direct loads issued before the first tiles' (the Q rows then wait for
  // nothing issued after them); V1's buffer holds the rows until V1 is loaded.
  lds_half *qs = lds + L::kBufBytes / 2;
  const bool rope = p.rope_cs != nullptr;
  const unsigned qstage = kt_a[0] + 3u * L::kTileHalfs * 2u;  // == vt_a[1]
  const unsigned csstage =
      lds_addr(lds + (L::kBufBytes + L::kQBytes + L::kMLBytes) / 2) + (unsigned)w * 1024u * NB;
  const int wq0 = tq0 + 2 * NB * w;  // first query of this wave's rows
#pragma unroll
  for (int j = 0; j < 4 * NB; ++j) {  // query j/2, heads 2(j&1) .. +1
    const int tq = min(wq0 + (j >> 1), p.S - 1);
    dma16(p.Q + (size_t)tq * dim_model + (size_t)(kvh * 4 + 2 * (j & 1)) * HD + 4 * lane,
          qstage + 1024u * j);
  }
  if (rope) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {  // queries 2j, 2j+1 of the wave
      const int tq = min(wq0 + 2 * j + (lane >> 5), p.S - 1);
      dma16(p.rope_cs + (size_t)tq * HD + 4 * (lane & 31), csstage + 1024u * j);
    }
  }
  issue_first_tiles();
  // the Q rows are in once at most the tile loads issued after them are pending
  if (g_count > 1) wait_vmcnt<24>();
  else if (g_count == 1) wait_vmcnt<16>();
  else wait_vmcnt<0>();
  u4 q_lo_keep[2 * NB];
#pragma unroll
  for (int k = 0; k < 2 * NB; ++k) {
    const int u = lane + 64 * k;
    const int rw = u >> 4, ch = u & 15;  // row within the wave's rows, 8-dim chunk
    const int rl = 8 * NB * w + rw;
    const int t = (row0 + rl) >> 2;
    const f4 a = *(const lds_f4 *)(__UINTPTR_TYPE__)(qstage + 512u * rw + 32u * ch);
    const f4 b = *(const lds_f4 *)(__UINTPTR_TYPE__)(qstage + 512u * rw + 32u * ch + 16u);
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (rope) {
      const unsigned ca = csstage + 512u * (rw >> 2) + 32u * ch;
      const f4 c0 = *(const lds_f4 *)(__UINTPTR_TYPE__)ca;
      const f4 c1 = *(const lds_f4 *)(__UINTPTR_TYPE__)(ca + 16u);
      rope_pair(v[0], v[1], c0.x, c0.y);
      rope_pair(v[2], v[3], c0.z, c0.w);
      rope_pair(v[4], v[5], c1.x, c1.y);
      rope_pair(v[6], v[7], c1.z, c1.w);
    }
    u4 packed = {0u, 0u, 0u, 0u}, packed_lo = {0u, 0u, 0u, 0u};
    if (t < p.S) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f2 x = {v[2 * e] * p.qscale, v[2 * e + 1] * p.qscale};
        const h2 hi = __builtin_convertvector(x, h2);
        const h2 lo = __builtin_convertvector(x - __builtin_convertvector(hi, f2), h2);
        packed[e] = __builtin_bit_cast(unsigned, hi);
        packed_lo[e] = __builtin_bit_cast(unsigned, lo);
      }
    }
    *(lds_u4 *)(qs + rl * HD + 8 * (ch ^ swz(rl))) = packed;
    q_lo_keep[k] = packed_lo;
  }
  __syncthreads();

  // Q^T operands: column = row, k-step st covers dims 16*st + 8*half .. +8;
  // the hi parts, then (through the same LDS rows) the lo parts.
  h8 qb[NB][8], ql[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int st = 0; st < 8; ++st)
      qb[b][st] = *(lds_h8 *)(qs + (32 * b + col) * HD + 8 * ((2 * st + half) ^ swz(col)));
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2 * NB; ++k) {
    const int u = lane + 64 * k;
    const int rw = u >> 4, ch = u & 15;
    const int rl = 8 * NB * w + rw;
    *(lds_u4 *)(qs + rl * HD + 8 * (ch ^ swz(rl))) = q_lo_keep[k];
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int st = 0; st < 8; ++st)
      ql[b][st] = *(lds_h8 *)(qs + (32 * b + col) * HD + 8 * ((2 * st + half) ^ swz(col)));

  // Softmax reference per row, fixed for the whole key range of the wave:
  // the max of the row's scores in its first tile (p <= 1 there), rounded to
  // fp16 and subtracted inside the score MFMA by one extra k-step (a ones
  // column in K against -m_ref in Q), so the loop neither subtracts nor
  // tracks maxima and never rescales the accumulators.  P's hi part is fp16,
  // so a later score more than ~16 (log2 units) above the reference
  // overflows it, and a row whose scores all sit far below an unset reference
  // underflows.  An underflowing row sums below 2^-8 (the fp32 row sum of the
  // unrounded P).  A P that rounds to fp16 infinity (>= 65520) makes the row
  // sum at least that and the row's accumulators non-finite (inf - inf from
  // its hi and lo parts); the accumulators are only inspected when the sum
  // is that large, so a long flat row with a large but finite sum costs one
  // look at them, not a second pass.  A wave with such a row sweeps its tiles
  // for the exact row maxima and runs once more with them as the reference.
  f16v o[NB][4];
  float m_ref[NB], l_run[NB];
  f16v s_cur[NB];
  h8 qx[NB];  // extra k-step B operand: -m_ref as fp16 hi, lo in elements 0, 1 of the half-0 lanes
#pragma unroll
  for (int b = 0; b < NB; ++b) m_ref[b] = -INFINITY;
  const h8 zero8 = {};
  h8 kx = {};  // extra k-step A operand: ones in k = 0, 1 for every key
  if (half == 0) {
    kx[0] = (_Float16)1.0f;
    kx[1] = (_Float16)1.0f;
  }
  auto set_ref = [&](int b, float m) {
    // m_ref = hi + lo (fp16 each): within ~2^-22 relative of m for |m| up to
    // ~1.2e5 log2 units, so P <= 1 holds at any realistic score magnitude (a
    // single fp16 would be off by up to 16 units beyond 32768); the applied
    // value is the one reported
    const float mc = m == -INFINITY ? 0.f : fminf(fmaxf(m, -1.2e5f), 1.2e5f);
    const _Float16 mh = (_Float16)fminf(fmaxf(mc, -6.0e4f), 6.0e4f);
    const _Float16 ml = (_Float16)(mc - (float)mh);
    m_ref[b] = m == -INFINITY ? -INFINITY : (float)mh + (float)ml;
    h8 x = {};
    if (half == 0) {
      x[0] = -mh;
      x[1] = -ml;
    }
    qx[b] = x;
  };

  // Tile kb needs masking unless every key is inside every row's window.
  auto needs_mask = [&](int kb) {
    bool m = kb + kKT > ke;
#pragma unroll
    for (int b = 0; b < NB; ++b)
      m = m || !bfull[b] || kb < lo_max[b] || kb + kKT - 1 > hi_min[b];
    return m;
  };
  // Keys outside the row's window, and keys before kb, become -inf; s[i] is
  // key kbl + (i/4)*8 + 4*half + (i%4) for the lane's row, kbl the tile's
  // first loaded key (kb except for a FAST kernel's last tile).
  // (The row bounds pass through an empty asm so that the compiler cannot
  // evaluate the per-score compares once for all tiles, ahead of the loop:
  // masks are rare, and the hoisted lane masks would be spilled.)
  auto mask_block = [&](f16v &s, int b, int kb, int kbl) {
    int lo = valid[b] ? max(lo_t[b], kb) - kbl - 4 * half : INT_MAX;
    int hi = min(hi_t[b], ke - 1) - kbl - 4 * half;
    asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int off = (i >> 2) * 8 + (i & 3);
      s[i] = off >= lo && off <= hi ? s[i] : -INFINITY;
    }
  };
  // The same when no row of the tile has its window's first key inside it
  // (kb >= lo_max of every block): only the upper edge, min(pos, ke - 1),
  // is left, one compare per score against a per-lane limit.
  auto mask_hi = [&](f16v &s, int b, int kb) {
    int hr = (valid[b] ? min(hi_t[b], ke - 1) : kb - 1) - kb - 4 * half;
    asm volatile("" : "+v"(hr));
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = (i >> 2) * 8 + (i & 3) <= hr ? s[i] : -INFINITY;
  };
  auto mask_tile = [&](f16v (&sc)[NB], int kb) {
    const int kbl = FAST ? min(kb, ke - kKT) : kb;
    bool lo_free = kbl == kb;
#pragma unroll
    for (int b = 0; b < NB; ++b) lo_free = lo_free && kb >= lo_max[b];
    if (lo_free) {
#pragma unroll
      for (int b = 0; b < NB; ++b) mask_hi(sc[b], b, kb);
    } else {
#pragma unroll
      for (int b = 0; b < NB; ++b) mask_block(sc[b], b, kb, kbl);
    }
  };
  // Row max of a score block over both key halves.
  auto block_max = [&](const f16v &s) {
    float m = fmaxf(s[0], s[1]);
#pragma unroll
    for (int i = 2; i < 16; i += 2) m = fmaxf(m, fmaxf(s[i], s[i + 1]));
    return half_swap_max(m);
  };
  // Unshifted scores of the tile in kt[buf] (first tile, max sweep).
  auto scores = [&](f16v (&sc)[NB], int buf, int kb) {
    h8 ka[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) ka[st] = lds_read_h8(ka_b[buf] ^ (unsigned)(st << 5));
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[b][i] = 0.f;
      mfma_qk_first(sc[b], ka[0], qb[b][0], ql[b][0]);
#pragma unroll
      for (int st = 1; st < 8; ++st) mfma_qk(sc[b], ka[st], qb[b][st], ql[b][st]);
    }
    qk_drain<NB>(sc);
    if (needs_mask(kb)) mask_tile(sc, kb);
  };

  // One tile step, with P.V one tile behind the scores: P of tile it from
  // s_cur (already shifted by the reference) into pb_next, shifted scores of
  // tile it+1 into s_cur, and (from it = 1 on) O += P.V of tile it-1 from
  // pb.  The MFMAs of a step (scores of it+1, P.V of it-1) are then
  // independent of the step's exponentials, which fill the issue slots
  // between them.  K(it+1) is in kt[(it+1)&1], V(it-1) in vt[(it+1)&1]; the
  // step refills kt[it&1] with K(it+2) at its start (K(it) was consumed by
  // the previous step) and vt[(it+1)&1] with V(it+1) after its P.V reads.
  // The K and V operands are streamed in halves (k-steps 0-3 / 4-7, keys
  // 0-15 / 16-31) to keep the register footprint within one wave per SIMD.
  // P^T of a tile as fp16 hi parts (keys 0-15, 16-31), then the lo parts.
  h8 pb[NB][4];
  // A single wave per SIMD issues everything in program order, so the step
  // is written in its issue order and fenced (sched_barrier) into small
  // groups: one or two MFMAs, then a slice of the exponentials, which then
  // execute on the VALU while the MFMAs run.
  auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
  auto step = [&](int it, auto with_pv) {
    const unsigned kab = ka_b[(it + 1) & 1];
    const unsigned vab = va_b[(it + 1) & 1];
    h8 ka[4], va[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) ka[st] = lds_read_h8(kab ^ (unsigned)(st << 5));
    if (with_pv) {
      va[0] = read_va<0, 0>(vab);
      va[1] = read_va<0, 1>(vab);
      va[2] = read_va<0, 2>(vab);
      va[3] = read_va<0, 3>(vab);
    }
    fence();
    // Exponential slice j (0 .. 4 NB - 1): scores 4(j%4) .. +3 of row block j/4.
    u4 pw[NB][4];  // hi parts (keys 0-15, 16-31), then lo parts
    float ls[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ls[b] = l_run[b];
    auto exp_slice = [&](int j) {
      const int b = j >> 2, i = 4 * (j & 3);
      const float p0 = fast_exp2(s_cur[b][i]), p1 = fast_exp2(s_cur[b][i + 1]);
      const float p2 = fast_exp2(s_cur[b][i + 2]), p3 = fast_exp2(s_cur[b][i + 3]);
      unsigned h0, l0, h1, l1;
      split_pair(p0, p1, h0, l0);
      split_pair(p2, p3, h1, l1);
      ls[b] = ((ls[b] + p0) + p1) + (p2 + p3);
      pw[b][i >> 3][(i & 7) >> 1] = h0;
      pw[b][i >> 3][((i & 7) >> 1) + 1] = h1;
      pw[b][2 + (i >> 3)][(i & 7) >> 1] = l0;
      pw[b][2 + (i >> 3)][((i & 7) >> 1) + 1] = l1;
      // used only by the next step: pinned here so that the work is not
      // sunk to the end of the step
      asm volatile("" ::"v"(h0), "v"(h1), "v"(l0), "v"(l1), "v"(ls[b]));
    };
    f16v s_next[NB];
    auto qk = [&](int st, int b) { mfma_qk(s_next[b], ka[st & 3], qb[b][st], ql[b][st]); };
    // scores of tile it+1: reference k-step, then k-steps 0-3
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s_next[b][i] = 0.f;
      s_next[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kx, qx[b], s_next[b], 0, 0, 0);
    }
    fence();
    exp_slice(0);
    fence();
#pragma unroll
    for (int b = 0; b < NB; ++b) qk(0, b);
    fence();
    // K(it) was consumed by the previous step: its buffer takes K(it+2)
    if (it + 2 < g_count) MIA_LOAD_K_NEXT(it + 2, it & 1);
    exp_slice(1);
    fence();
#pragma unroll
    for (int b = 0; b < NB; ++b) qk(1, b);
    fence();
    exp_slice(2);
    fence();
#pragma unroll
    for (int b = 0; b < NB; ++b) qk(2, b);
    fence();
    exp_slice(3);
    fence();
#pragma unroll
    for (int b = 0; b < NB; ++b) qk(3, b);
    fence();
#pragma unroll
    for (int st = 0; st < 4; ++st) ka[st] = lds_read_h8(kab ^ (unsigned)((st + 4) << 5));
    fence();
    // P.V of tile it-1, keys 0-15, interleaved with the rest of the slices
    int sl = 4;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      if (with_pv) {
#pragma unroll
        for (int b = 0; b < NB; ++b) mfma_pv2(o[b][db], va[db], pb[b][0], pb[b][2]);
      }
      fence();
      if (sl < 4 * NB) exp_slice(sl);  // NB = 1 has four slices only
      ++sl;
      fence();
    }
    if (with_pv) {
      va[0] = read_va<1, 0>(vab);
      va[1] = read_va<1, 1>(vab);
      va[2] = read_va<1, 2>(vab);
      va[3] = read_va<1, 3>(vab);
    }
    fence();
    // k-steps 4-7 and P.V keys 16-31, alternating
#pragma unroll
    for (int st = 4; st < 8; ++st) {
#pragma unroll
      for (int b = 0; b < NB; ++b) qk(st, b);
      if (with_pv) {
#pragma unroll
        for (int b = 0; b < NB; ++b) mfma_pv2(o[b][st - 4], va[st - 4], pb[b][1], pb[b][3]);
      }
      fence();
    }
    qk_drain<NB>(s_next);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      l_run[b] = ls[b];
#pragma unroll
      for (int h = 0; h < 4; ++h) pb[b][h] = __builtin_bit_cast(h8, pw[b][h]);
    }
    if (it + 1 < g_count) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // V(it-1) reads done
      MIA_LOAD_V_NEXT(it + 1, (it + 1) & 1);
    }
    // Window mask of tile it+1, only where it crosses a window edge.
    const int kbn = kb0 + kStride * (it + 1);
    if (needs_mask(kbn)) mask_tile(s_next, kbn);
#pragma unroll
    for (int b = 0; b < NB; ++b) s_cur[b] = s_next[b];
  };
  // O += P.V of the wave's last tile (its V in vt[(g_count-1)&1]).
  auto last_pv = [&]() {
    const unsigned vab = va_b[(g_count - 1) & 1];
    h8 va[4];
    va[0] = read_va<0, 0>(vab);
    va[1] = read_va<0, 1>(vab);
    va[2] = read_va<0, 2>(vab);
    va[3] = read_va<0, 3>(vab);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int b = 0; b < NB; ++b) mfma_pv2(o[b][db], va[db], pb[b][0], pb[b][2]);
    va[0] = read_va<1, 0>(vab);
    va[1] = read_va<1, 1>(vab);
    va[2] = read_va<1, 2>(vab);
    va[3] = read_va<1, 3>(vab);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int b = 0; b < NB; ++b) mfma_pv2(o[b][db], va[db], pb[b][1], pb[b][3]);
  };

  // NB = 2 (prefill): the same step as 34 slots of one score k-step (hi and
  // lo q) or one P.V k-step (hi and lo P), i.e. two MFMAs, except the two
  // reference k-steps; each slot is followed by one exponential of tile it
  // (with its hi + lo split and row-sum work every second slot), so the
  // transcendental issue sits under the MFMAs instead of the exponentials
  // queueing behind half of them.
  // Scores and P live in two register sets that alternate between steps
  // (s_in -> s_out, p_in -> p_out), so nothing is copied at the step's end.
  // with_qk is false for a wave's last tile, whose step has no next tile to
  // score: its slots then hold only the exponentials and the P.V MFMAs.
  auto step2 = [&](int it, auto with_pv, auto with_qk, f16v(&s_in)[NB], f16v(&s_out)[NB],
                   h8(&p_in)[NB][4], h8(&p_out)[NB][4]) {
    const unsigned kab = ka_b[(it + 1) & 1];
    const unsigned vab = va_b[(it + 1) & 1];
    // Operands in halves, each read eight slots (~256 cycles) ahead of its
    // first use: K k-steps 0-3 and V^T keys 0-15 now, k-steps 4-7 in slot 11,
    // V^T keys 16-31 in slot 19 (into the registers the first halves free).
    h8 ka[8], vlo[4], vhi[4];
    if (with_qk) {
#pragma unroll
      for (int st = 0; st < 4; ++st) ka[st] = lds_read_h8(kab ^ (unsigned)(st << 5));
    }
    if (with_pv) {
      vlo[0] = read_va<0, 0>(vab);
      vlo[1] = read_va<0, 1>(vab);
      vlo[2] = read_va<0, 2>(vab);
      vlo[3] = read_va<0, 3>(vab);
    }
    fence();
    float ls[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ls[b] = l_run[b];
    u4 pw[NB][4];  // hi parts (keys 0-15, 16-31), then lo parts
    float ex[4];
    // Element k of exponential slice j: score e = 4 (j % 4) + k of row block
    // j / 4; odd k splits the pair (e-1, e) into fp16 hi and lo parts and
    // adds it to the sum.
    // (The results are pinned where they are formed: they are only read at
    // the step's end, and would otherwise be sunk there, behind the MFMAs.)
    auto E = [&](int j, int k) {
      const int b = j >> 2, e = 4 * (j & 3) + k;
      ex[k] = fast_exp2(s_in[b][e]);
      ls[b] += ex[k];
      if (k & 1) {
        unsigned hi, lo;
        split_pair(ex[k - 1], ex[k], hi, lo);
        pw[b][e >> 3][((e - 1) & 7) >> 1] = hi;
        pw[b][2 + (e >> 3)][((e - 1) & 7) >> 1] = lo;
        asm volatile("" ::"v"(hi), "v"(lo), "v"(ls[b]));
      } else {
        asm volatile("" ::"v"(ex[k]), "v"(ls[b]));
      }
    };
    auto REF = [&](int b) {
      if (!with_qk) return;
      f16v z;
#pragma unroll
      for (int i = 0; i < 16; ++i) z[i] = 0.f;
      s_out[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kx, qx[b], z, 0, 0, 0);
    };
    auto QK = [&](int st, int b) {
      if (with_qk) mfma_qk(s_out[b], ka[st], qb[b][st], ql[b][st]);
    };
    auto PVL = [&](int db, int b) {
      if (with_pv) mfma_pv2(o[b][db], vlo[db], p_in[b][0], p_in[b][2]);
    };
    auto PVH = [&](int db, int b) {
      if (with_pv) mfma_pv2(o[b][db], vhi[db], p_in[b][1], p_in[b][3]);
    };
    // slots 1-10: reference k-steps and k-steps 0-3; exponential slices 0-2
    REF(0); fence(); E(0, 0); fence();
    REF(1); fence(); E(0, 1); fence();
    QK(0, 0); fence(); E(0, 2); fence();
    QK(0, 1); fence(); E(0, 3); fence();
    // K(it) was consumed by the previous step: its buffer takes K(it+2)
    QK(1, 0); fence(); E(1, 0);
    if (it + 2 < g_count) MIA_LOAD_K_NEXT(it + 2, it & 1);
    fence();
    QK(1, 1); fence(); E(1, 1); fence();
    QK(2, 0); fence(); E(1, 2); fence();
    QK(2, 1); fence(); E(1, 3); fence();
    QK(3, 0); fence(); E(2, 0); fence();
    QK(3, 1); fence(); E(2, 1); fence();
    // The P.V MFMAs are inline assembly, so the compiler does not know how
    // long they read their V^T and P registers: a register whose last reader
    // is one of them is kept alive (keep) past the next slot's MFMA, one MFMA
    // duration later, before anything may be written into it.  Each slot's
    // MFMA (and keep) is fenced off from its exponential, which the compiler
    // would otherwise place first.
    auto keep = [&](const h8 &x) {
      if (with_pv) asm volatile("" ::"v"(x));
    };
    // slots 11-18: P.V of tile it-1, keys 0-15
    if (with_qk) {
#pragma unroll
      for (int st = 4; st < 8; ++st) ka[st] = lds_read_h8(kab ^ (unsigned)(st << 5));
    }
    PVL(0, 0); fence(); E(2, 2); fence();
    PVL(0, 1); fence(); E(2, 3); fence();
    PVL(1, 0); keep(vlo[0]); fence(); E(3, 0); fence();
    PVL(1, 1); fence(); E(3, 1); fence();
    PVL(2, 0); keep(vlo[1]); fence(); E(3, 2); fence();
    PVL(2, 1); fence(); E(3, 3); fence();
    PVL(3, 0); keep(vlo[2]); fence(); E(4, 0); fence();
    PVL(3, 1); fence(); E(4, 1); fence();
    // slots 19-26: k-steps 4-7
    QK(4, 0);
    keep(vlo[3]);
    keep(p_in[0][0]);
    keep(p_in[1][0]);
    keep(p_in[0][2]);
    keep(p_in[1][2]);
    fence();
    if (with_pv) {
      vhi[0] = read_va<1, 0>(vab);
      vhi[1] = read_va<1, 1>(vab);
      vhi[2] = read_va<1, 2>(vab);
      vhi[3] = read_va<1, 3>(vab);
    }
    E(4, 2); fence();
    QK(4, 1); fence(); E(4, 3); fence();
    QK(5, 0); fence(); E(5, 0); fence();
    QK(5, 1); fence(); E(5, 1); fence();
    QK(6, 0); fence(); E(5, 2); fence();
    QK(6, 1); fence(); E(5, 3); fence();
    QK(7, 0); fence(); E(6, 0); fence();
    QK(7, 1); fence(); E(6, 1);
    if (with_qk) qk_drain<NB>(s_out);
    fence();
    // slots 27-34: P.V keys 16-31; V(it+1) goes into V(it-1)'s buffer once
    // every LDS read of the step is done
    PVH(0, 0); fence(); E(6, 2); fence();
    PVH(0, 1); fence(); E(6, 3); fence();
    PVH(1, 0); keep(vhi[0]); fence(); E(7, 0); fence();
    PVH(1, 1); fence(); E(7, 1); fence();
    PVH(2, 0); keep(vhi[1]); fence(); E(7, 2); fence();
    PVH(2, 1); fence(); E(7, 3); fence();
    PVH(3, 0);
    keep(vhi[2]);
    fence();
    if (it + 1 < g_count) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      MIA_LOAD_V_NEXT(it + 1, (it + 1) & 1);
    }
    fence();
    PVH(3, 1);
    // The P.V MFMAs are inline assembly: the compiler neither sees that they
    // write the accumulators nor pads what it places after them.  Wait for
    // their results here, so that no register copy it may insert later (at
    // a loop edge or a branch join) reads an accumulator still in flight.
    if (with_pv) pv_drain_all(o);
    fence();
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      l_run[b] = ls[b];
#pragma unroll
      for (int h = 0; h < 4; ++h) p_out[b][h] = __builtin_bit_cast(h8, pw[b][h]);
    }
    // Window mask of tile it+1, only where it crosses a window edge.
    if (with_qk) {
      const int kbn = kb0 + kStride * (it + 1);
      if (needs_mask(kbn)) mask_tile(s_out, kbn);
    }
  };
  // O += P.V of the wave's last tile (its V in vt[(g_count-1)&1]) from P.
  // The MFMAs are inline assembly, invisible to the compiler's hazard
  // checks: the leading wait states keep them from reading P registers the
  // step just wrote.
  auto last_pv_of = [&](h8(&pl)[NB][4]) {
    asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
    const unsigned vab = va_b[(g_count - 1) & 1];
    h8 va[4];
    va[0] = read_va<0, 0>(vab);
    va[1] = read_va<0, 1>(vab);
    va[2] = read_va<0, 2>(vab);
    va[3] = read_va<0, 3>(vab);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int b = 0; b < NB; ++b) mfma_pv2(o[b][db], va[db], pl[b][0], pl[b][2]);
    va[0] = read_va<1, 0>(vab);
    va[1] = read_va<1, 1>(vab);
    va[2] = read_va<1, 2>(vab);
    va[3] = read_va<1, 3>(vab);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int b = 0; b < NB; ++b) mfma_pv2(o[b][db], va[db], pl[b][1], pl[b][3]);
    pv_drain_all(o);
  };

  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) {
      // Exact row maxima over the wave's tiles, then the same pass again.
      float mt[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) mt[b] = -INFINITY;
      for (int i = 0; i < g_count; ++i) {
        MIA_LOAD_K(i, 0);
        wait_vmcnt<0>();
        f16v sc[NB];
        scores(sc, 0, kb0 + kStride * i);
#pragma unroll
        for (int b = 0; b < NB; ++b) mt[b] = fmaxf(mt[b], block_max(sc[b]));
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) set_ref(b, mt[b]);
      issue_first_tiles();
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int db = 0; db < 4; ++db) mfma_zero(o[b][db], zero8);
      l_run[b] = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) s_cur[b][i] = -INFINITY;
    }
    // The first tile's scores set the reference (first pass) and are
    // shifted by it.
    if (g_count > 0) {
      if (g_count > 1) wait_vmcnt<16>();  // K1 and V0 may be pending
      else wait_vmcnt<8>();
      scores(s_cur, 0, kb0);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (pass == 0) set_ref(b, block_max(s_cur[b]));
        const float sh = m_ref[b] == -INFINITY ? 0.f : m_ref[b];
#pragma unroll
        for (int i = 0; i < 16; ++i) s_cur[b][i] -= sh;
      }
    } else {
#pragma unroll
      for (int b = 0; b < NB; ++b) set_ref(b, -INFINITY);
    }

    // Loads are issued in the order K0 K1 V0 | K2 V1 | K3 V2 | ... (step it
    // issues K(it+2), then V(it+1)).  Step it needs K(it+1) and V(it-1): only
    // V(it), the last load issued, may still be pending.
    if constexpr (NB == 2) {
      // Step it exponentiates tile it and scores tile it+1; the last step
      // (it = g_count - 1) scores nothing.
      using T = std::true_type;
      using F = std::false_type;
      f16v s_alt[NB];
      h8 p_a[NB][4], p_b[NB][4];
      if (g_count > 0) {
        wait_vmcnt<8>();
        step2(0, F{}, T{}, s_cur, s_alt, p_a, p_b);  // P(0) -> p_b
      }
      int it = 1;
      for (; it + 2 < g_count; it += 2) {
        wait_vmcnt<8>();
        step2(it, T{}, T{}, s_alt, s_cur, p_b, p_a);
        wait_vmcnt<8>();
        step2(it + 1, T{}, T{}, s_cur, s_alt, p_a, p_b);
      }
      if (it + 1 < g_count) {  // it = g_count - 2: one more scoring step
        wait_vmcnt<8>();
        step2(it, T{}, T{}, s_alt, s_cur, p_b, p_a);
        ++it;
#pragma unroll
        for (int b = 0; b < NB; ++b) {  // into the registers the last step reads
          s_alt[b] = s_cur[b];
#pragma unroll
          for (int h = 0; h < 4; ++h) p_b[b][h] = p_a[b][h];
        }
      }
      if (it < g_count) {  // it = g_count - 1: the last step
        wait_vmcnt<8>();
        step2(it, T{}, F{}, s_alt, s_cur, p_b, p_a);
#pragma unroll
        for (int b = 0; b < NB; ++b) {  // P of the last tile where last_pv_of reads it
#pragma unroll
          for (int h = 0; h < 4; ++h) p_b[b][h] = p_a[b][h];
        }
      }
      if (g_count > 0) {
        wait_vmcnt<0>();
        last_pv_of(p_b);
      }
    } else {
      if (g_count > 0) {
        wait_vmcnt<8>();
        step(0, std::false_type{});
      }
      for (int it = 1; it < g_count; ++it) {
        wait_vmcnt<8>();
        step(it, std::true_type{});
      }
      if (g_count > 0) {
        wait_vmcnt<0>();
        last_pv();
      }
    }
    // Row sums: an underflow (< 2^-8 with keys in range, or not finite) means
    // the reference did not suit the row; so does an fp16 overflow of some P,
    // possible only where the sum reaches 65504 and then visible as a
    // non-finite accumulator of the row.
    bool bad = false, large = false;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float lt = half_swap_sum(l_run[b]);
      l_run[b] = lt;
      bad = bad || (has_keys[b] && !(lt >= 0.00390625f));
      large = large || (has_keys[b] && !(lt < 65504.0f));
    }
    if (pass == 0 && __builtin_amdgcn_ballot_w64(large) != 0) {
      pv_drain<NB>(o);
      bool nonfinite = false;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        // a sum of the row's accumulators is non-finite iff one of them is
        // (at magnitudes far below fp32's range)
        float t = 0.f;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) t += o[b][db][i];
        t = half_swap_sum(t);
        nonfinite = nonfinite || (has_keys[b] && !__builtin_isfinite(t));
      }
      bad = bad || nonfinite;
    }
    if (pass == 1 || __builtin_amdgcn_ballot_w64(bad) == 0) break;
  }
#undef MIA_LOAD_FAST
#undef MIA_LOAD_K
#undef MIA_LOAD_V
#undef MIA_LOAD_K_NEXT
#undef MIA_LOAD_V_NEXT

  // ---- merge of the four key groups ----
  // Each wave leaves its (max, sum) per row and its unscaled partial output
  // in its own tile buffers, which are free once its loop is done (its loads
  // have landed; its reads of them come first in its LDS order): a wave that
  // finishes early writes without waiting for the others.  After one
  // barrier, wave w finalises dim block w of every row block from the four
  // partials, weighted by e_k = 2^(m_k - M): its own from its registers, the
  // other three from LDS, lane-linear (conflict-free).
  pv_drain<NB>(o);
  lds_float *ml = (lds_float *)(smem + L::kBufBytes + L::kQBytes);  // [wave][RT][2]
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    // reference actually applied: m_ref, or 0 where it stayed unset although
    // the row has keys here; rows without keys get weight 0 in the merge
    const float mr = !has_keys[b] ? -INFINITY : (m_ref[b] == -INFINITY ? 0.f : m_ref[b]);
    if (half == 0) *(lds_f2 *)(ml + (w * RT + 32 * b + col) * 2) = (f2){mr, l_run[b]};
  }
  // wave src's partial of (row block b, dim block db), chunk q of this lane
  constexpr int kWaveBufBytes = L::kBufBytes / kWaves;
  static_assert(NB * 4 * 4 * 64 * 16 <= kWaveBufBytes, "a wave's partial must fit its tile buffers");
  auto mg_at = [&](int src, int b, int db, int q) {
    return (lds_float *)(smem + src * kWaveBufBytes) + (((b * 4 + db) * 4 + q) * 64 + lane) * 4;
  };
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      if (db == w) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *(lds_f4 *)mg_at(w, b, db, q) =
            (f4){o[b][db][4 * q], o[b][db][4 * q + 1], o[b][db][4 * q + 2], o[b][db][4 * q + 3]};
    }
  __syncthreads();

  const size_t tile_id = (size_t)kvh * p.n_rtiles + rtile;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    f2 mlw[kWaves];
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      mlw[k] = *(lds_f2 *)(ml + (k * RT + 32 * b + col) * 2);
      M = fmaxf(M, mlw[k].x);
    }
    float e[kWaves], Ls = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      e[k] = mlw[k].x == -INFINITY ? 0.f : fast_exp2(mlw[k].x - M);
      Ls = __builtin_fmaf(e[k], mlw[k].y, Ls);
    }
    const int rl = 32 * b + col;
    const int row = row0 + rl;
    const int t = row >> 2, g = row & 3;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      if (db != w) continue;
      f4 acc[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[q] = (f4){o[b][db][4 * q], o[b][db][4 * q + 1], o[b][db][4 * q + 2], o[b][db][4 * q + 3]} *
                 e[db];
#pragma unroll
        for (int k = 0; k < kWaves; ++k)
          if (k != db) acc[q] += *(lds_f4 *)mg_at(k, b, db, q) * e[k];
      }
      if (t < p.S) {
        // dims 32*db + 8*q + 4*half .. +4 (the accumulator's dim order)
        if (p.nsplit == 1) {
          const float inv = 1.0f / Ls;
          float *dst = p.out + (size_t)t * dim_model + (size_t)(kvh * 4 + g) * HD + 32 * db + 4 * half;
#pragma unroll
          for (int q = 0; q < 4; ++q) *reinterpret_cast<f4 *>(dst + 8 * q) = acc[q] * inv;
        } else {
          const size_t pidx = (tile_id * p.nsplit + split) * RT + rl;
          float *dst = p.part_o + pidx * HD + 32 * db + 4 * half;
#pragma unroll
          for (int q = 0; q < 4; ++q) *reinterpret_cast<f4 *>(dst + 8 * q) = acc[q];
          if (db == 0 && half == 0)
            *reinterpret_cast<float2 *>(p.part_ml + pidx * 2) = make_float2(M, Ls);
        }
      }
    }
  }
}

// Split merge: one workgroup per row of a tile.  Thread = (split group sg of
// 32, 16 dims): it holds splits sg, sg+32, ... of its dims, all loaded before
// the first reduction (one memory round trip however many splits there
// are), then the splits are reduced through LDS.  With p.commit_k set, the
// first S workgroups also copy the staged drafts into their ring slots: the
// kernel boundary orders that after every read of the ring by the attention
// kernel.  A separate launch, so the boundary also orders the partial writes
// before these reads.
constexpr int kMergeSplitsPerThread = 8;  // 256 splits at most
__global__ void __launch_bounds__(256) flash_merge_kernel(FlashParams p, int rt) {
  __shared__ float red[32][HD + 4];
  __shared__ float wmax[4], wsum[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int kv_dim = p.n_kv * HD;
  // (rows t < S - max_seq are overwritten by later rows in the same slot)
  if (p.commit_k != nullptr && (int)blockIdx.x < p.S && (int)blockIdx.x >= p.S - p.max_seq) {
    const int t = blockIdx.x;
    const size_t slot = (size_t)((p.start_pos + t) % p.max_seq);
    for (int e = 4 * tid; e < kv_dim; e += 4 * 256) {
      *reinterpret_cast<uint2 *>(p.commit_k + slot * kv_dim + e) =
          *reinterpret_cast<const uint2 *>(p.kstage + (size_t)t * kv_dim + e);
      *reinterpret_cast<uint2 *>(p.commit_v + slot * kv_dim + e) =
          *reinterpret_cast<const uint2 *>(p.vstage + (size_t)t * kv_dim + e);
    }
  }
  if ((int)blockIdx.x >= p.n_kv * p.n_rtiles * rt) return;  // commit-only workgroup
  const int tile_id = blockIdx.x / rt, rl = blockIdx.x % rt;
  const int kvh = tile_id / p.n_rtiles, rtile = tile_id % p.n_rtiles;
  const int row = rtile * rt + rl;
  const int t = row >> 2, g = row & 3;
  if (t >= p.S) return;  // whole workgroup
  const int sg = tid >> 3, d16 = tid & 7;
  const size_t base = (size_t)tile_id * p.nsplit * rt + rl;  // + sp * rt
  float m[kMergeSplitsPerThread], l[kMergeSplitsPerThread];
  f4 o[kMergeSplitsPerThread][4];
#pragma unroll
  for (int k = 0; k < kMergeSplitsPerThread; ++k) {
    const int sp = sg + 32 * k;
    m[k] = -INFINITY;
    l[k] = 0.f;
    if (sp < p.nsplit) {
      const size_t idx = base + (size_t)sp * rt;
      const float2 ml = *reinterpret_cast<const float2 *>(p.part_ml + idx * 2);
      m[k] = ml.x;
      l[k] = ml.y;
      const f4 *src = reinterpret_cast<const f4 *>(p.part_o + idx * HD + 16 * d16);
#pragma unroll
      for (int q = 0; q < 4; ++q) o[k][q] = src[q];
    }
  }
  float M = m[0];
#pragma unroll
  for (int k = 1; k < kMergeSplitsPerThread; ++k) M = fmaxf(M, m[k]);
  M = wave_max(M);
  if (lane == 0) wmax[wv] = M;
  __syncthreads();
  M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float Mu = M == -INFINITY ? 0.f : M;
  f4 acc[4] = {};
  float ls = 0.f;
#pragma unroll
  for (int k = 0; k < kMergeSplitsPerThread; ++k) {
    if (sg + 32 * k < p.nsplit) {
      const float e = m[k] == -INFINITY ? 0.f : fast_exp2(m[k] - Mu);
      ls = __builtin_fmaf(e, l[k], ls);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] += e * o[k][q];
    }
  }
  // every split's l is held by the 8 threads of its group: count it once
  ls = wave_sum(d16 == 0 ? ls : 0.f);
  if (lane == 0) wsum[wv] = ls;
#pragma unroll
  for (int q = 0; q < 4; ++q) *reinterpret_cast<f4 *>(&red[sg][16 * d16 + 4 * q]) = acc[q];
  __syncthreads();
  if (tid < HD) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) sum += red[k][tid];
    const float Ls = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    p.out[(size_t)t * (kv_dim * 4) + (size_t)(kvh * 4 + g) * HD + tid] = sum / Ls;
  }
}

template <int NB, bool FAST>
hipError_t set_lds_limit() {
  return hipFuncSetAttribute((const void *)flash_kernel<NB, FAST>,
                             hipFuncAttributeMaxDynamicSharedMemorySize, Lay<NB>::kBytes);
}

int rows_per_tile(int S) { return S * 4 <= 32 ? 32 : 64; }

// The FAST kernel's conditions: no staged rows, no key split, no window
// reaching past the ring's end (every row's window starts at key 0 and no
// tile wraps), and every workgroup's key range at least one tile long (the
// shortest is the first row tile's, start_pos + its query count).
bool flash_fast_ok(const FlashParams &p) {
  const int first_rows = rows_per_tile(p.S) / 4;
  return p.kstage == nullptr && p.vstage == nullptr && p.nsplit == 1 &&
         (long)p.start_pos + p.S <= (long)p.max_seq &&
         (long)p.start_pos + (p.S < first_rows ? p.S : first_rows) >= kKT;
}

template <int NB>
hipError_t launch_variant(const FlashParams &p, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  using L = Lay<NB>;
  dim3 grid(p.n_kv * p.n_rtiles * p.nsplit);
  if (flash_fast_ok(p))
    hipExtLaunchKernelGGL((flash_kernel<NB, true>), grid, dim3(256), L::kBytes, s, ev0, ev1, 0, p);
  else
    hipExtLaunchKernelGGL((flash_kernel<NB, false>), grid, dim3(256), L::kBytes, s, ev0, ev1, 0,
                          p);
  return hipGetLastError();
}

}  // namespace

hipError_t prepare_flash() {
  hipError_t e = set_lds_limit<1, false>();
  if (e == hipSuccess) e = set_lds_limit<2, false>();
  if (e == hipSuccess) e = set_lds_limit<1, true>();
  return e != hipSuccess ? e : set_lds_limit<2, true>();
}

size_t flash_scratch_bytes(int n_kv, int n_rtiles, int nsplit, int rows_per_tile) {
  return (size_t)n_kv * n_rtiles * nsplit * rows_per_tile * (HD + 2) * sizeof(float);
}

// Few rows (S*G <= 32, e.g. speculative verify): one 32-row block, key splits
// over workgroups until about target_wgs workgroups.  Otherwise (prefill):
// 64-row tiles, no split unless the row tiles alone leave the device mostly
// idle.  Every wave of a split keeps at least 4 tiles of 32 keys.
void flash_plan(int S, int n_kv, int G, int start_pos, int max_seq, int target_wgs, int *n_rtiles,
                int *nsplit, int *split_keys, int *rows_per_tile_out) {
  const int rt = rows_per_tile(S);
  const int ntiles = (S * G + rt - 1) / rt;
  long maxkeys = 0;
  for (int ti = 0; ti < ntiles; ++ti) {
    int t0 = (ti * rt) / G;
    int t1 = ((ti + 1) * rt - 1) / G;
    if (t1 > S - 1) t1 = S - 1;
    long p0 = (long)start_pos + t0;
    long lo = p0 + 1 > max_seq ? p0 + 1 - max_seq : 0;
    long hi = (long)start_pos + t1;
    if (hi - lo + 1 > maxkeys) maxkeys = hi - lo + 1;
  }
  long want = (long)target_wgs / ((long)n_kv * ntiles);
  if (want < 1) want = 1;
  long max_split = maxkeys / (4L * kWaves * kKT);
  if (max_split > kMergeSplitsPerThread * 32) max_split = kMergeSplitsPerThread * 32;
  if (want > max_split) want = max_split > 0 ? max_split : 1;
  long sk = (maxkeys + want - 1) / want;
  sk = ((sk + kKT - 1) / kKT) * kKT;
  long ns = (maxkeys + sk - 1) / sk;
  if (ns < 1) ns = 1;
  *n_rtiles = ntiles;
  *nsplit = (int)ns;
  *split_keys = (int)sk;
  *rows_per_tile_out = rt;
}

hipError_t launch_flash(const FlashParams &p, int G, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (G != 4) return hipErrorInvalidValue;
  return rows_per_tile(p.S) == 32 ? launch_variant<1>(p, s, ev0, ev1)
                                  : launch_variant<2>(p, s, ev0, ev1);
}

hipError_t launch_flash_merge(const FlashParams &p, hipStream_t s) {
  const int rt = rows_per_tile(p.S);
  if (p.nsplit > kMergeSplitsPerThread * 32) return hipErrorInvalidValue;
  if (p.nsplit > 1) {
    // one workgroup per row; with a commit, at least S of them
    const int wgs = max(p.n_kv * p.n_rtiles * rt, p.commit_k != nullptr ? p.S : 0);
    hipLaunchKernelGGL(flash_merge_kernel, dim3(wgs), dim3(256), 0, s, p, rt);
  }
  return hipGetLastError();
}

}  // namespace mia
