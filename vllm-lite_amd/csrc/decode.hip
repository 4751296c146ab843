// Single-token decode attention over the paged KV cache (pa_decode).
//
// Work split (flash-decoding): the context of each sequence is cut into
// partitions (kPart tokens, or longer for the MFMA kernel when that streams
// faster; see choose_partition).  One workgroup handles one (partition,
// kv head, sequence) and produces, for each query head of the group, the
// running max m (log2 domain), the softmax denominator l and the
// unnormalised output o[D].  A single-partition launch writes the final
// output directly; otherwise a reduce kernel merges the partitions with the
// log-sum-exp rule
//     M = max_p m_p,  out = sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M) l_p.
//
// Two attention kernels:
//  * decode_mfma_kernel (bf16, D in {64, 128, 256}, group size <= 16): one
//    wavefront per workgroup.  Scores S = K·Qᵀ and the output Oᵀ = Vᵀ·Pᵀ
//    both run on v_mfma_f32_16x16x32_bf16 with the query heads of the group
//    as the 16-wide N dimension, so every K/V byte is loaded once for the
//    whole group.  Loads go straight from HBM into MFMA operand registers:
//    K rows are token-major, V rows are token-minor, which is exactly the
//    operand order each contraction wants.  Two 16-token blocks are
//    processed per step (32 = the MFMA K dimension of the P·V product).
//  * decode_generic_kernel (f32 or bf16, any D <= 512, any group size): a
//    plain reference-grade kernel, one workgroup per query head.
#include <mutex>
#include <type_traits>

#include "pa_common.hpp"
#include "pa_internal.hpp"

namespace pa {
namespace {

// Tokens per partition.  The generic kernel always uses kPart; the MFMA
// kernel picks a multiple of it per launch (choose_partition).
constexpr int kPart = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;  // "no max yet": finite so 2^(x - m) never sees inf - inf

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline float shfl_xor_f(float x, int mask) { return __shfl_xor(x, mask, 64); }

// K/V of a block that only this sequence reads are streamed once per decode
// step: non-temporal loads (the `nt` cache policy) keep them from
// displacing reusable lines and stream faster (measured ~6.8 TB/s vs
// ~6.1 TB/s for plain 16-byte loads on MI355X).  Blocks that a neighbouring
// sequence's table holds at the same index (a shared prefix) are read with
// the default policy, so the other sequences find them in the cache.
// The loads are raw buffer loads over one (block, head) slice, whose cache
// policy is an instruction operand (a select between a plain and a
// non-temporal pointer load would be merged into a plain load).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kPolicyNT = 2;  // cache-policy operand: non-temporal
__device__ inline __amdgpu_buffer_rsrc_t slice_rsrc(const void* base, int bytes) {
  // raw buffer (stride 0) of `bytes` bytes; 32-bit data format, so reads past
  // the slice return zeros
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
template <int POLICY>
__device__ inline u32x4 bload16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POLICY);
}
template <int POLICY>
__device__ inline uint64_t bload8(__amdgpu_buffer_rsrc_t r, int off) {
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POLICY);
  return (uint64_t)v[0] | ((uint64_t)v[1] << 32);
}
// Whether table entry `bi` of sequence `seq` is private to it: the tables
// of the sequences before and after hold a different block at that index.
__device__ inline bool private_block(const int32_t* __restrict__ block_tables, int mbs, int seq,
                                     int num_seqs, int bi, int32_t id) {
  const bool prev = seq > 0 && block_tables[(int64_t)(seq - 1) * mbs + bi] == id;
  const bool next = seq + 1 < num_seqs && block_tables[(int64_t)(seq + 1) * mbs + bi] == id;
  return !prev && !next;
}

// Merge of the partial results held by the NW wavefronts of a workgroup,
// one partition each, together all partitions of one (kv head, sequence):
// through LDS, with the log-sum-exp rule of decode_reduce_kernel
//     M = max_w m_w,  out = sum_w 2^(m_w - M) o_w / sum_w 2^(m_w - M) l_w,
// written as the bf16 output of the group's G query heads (empty partitions
// hold m = kNegBig, l = 0, o = 0 and drop out).  Lane (c, j) holds head c's
// o[dt][r] for dims 16 dt + 4 j + r, as the MFMA decode kernels leave it.
template <int D, int NW>
__device__ inline void merge_in_workgroup(uint16_t* __restrict__ out_group, const f32x4 (&o)[D / 16],
                                          float m, float lsum, int c, int j, int G) {
  __shared__ float so[NW][16][D];
  __shared__ float sml[NW][16][2];
  const int wave = threadIdx.x >> 6;
  if (c < G) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) so[wave][c][16 * dt + 4 * j + r] = o[dt][r];
    if (j == 0) {
      sml[wave][c][0] = m;
      sml[wave][c][1] = lsum;
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += 64 * NW) {
    const int hc = idx / D, d = idx % D;
    float mx = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, sml[w][hc][0]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = fast_exp2(sml[w][hc][0] - mx);
      num += a * so[w][hc][d];
      den += a * sml[w][hc][1];
    }
    // den is 0 only for a row with no keys; a NaN den (a NaN score) must
    // reach the output, so the test is != 0, not > 0
    out_group[idx] = f32_to_bf16_bits(den != 0.f ? num / den : 0.f);
  }
}

// ---------------------------------------------------------------------------
// MFMA decode kernel.
//
// Lane layout (lane = 16 * j + c, c = lane & 15, j = lane >> 4), using the
// v_mfma_f32_16x16x32_bf16 operand layouts
//   A[i][k]: lane holds row i = c, k = 8j .. 8j+7
//   B[k][n]: lane holds col n = c, k = 8j .. 8j+7
//   D[i][n]: lane holds col n = c, rows i = 4j .. 4j+3
// QK:  A = K block (i = token c), B = Qᵀ (n = head c of the group), the
//      D = 128 reduction split in 32-wide steps s, lane group j taking dims
//      32s + 8j .. +8 in both operands.  Result: lane holds S[token 4j+r][head c].
// PV:  A = Vᵀ (i = dim 16dt + c), B = Pᵀ (n = head c); the 32 reduction slots
//      8j+r / 8j+4+r are tokens 4j+r of the first / second block of the step,
//      which is exactly what the lane already holds from QK.  Result: lane
//      holds Oᵀ[dim 16dt + 4j + r][head c].
template <int D, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void decode_mfma_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ context_lens, int Hq, int Hkv, int G, int num_blocks,
    float scale_log2, int num_parts, int part_len, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, int64_t q_row, const uint8_t* /* FP8 flags, unused */) {
  constexpr int KS = D / 32;  // QK reduction steps
  constexpr int DT = D / 16;  // PV output tiles
  // NW > 1: the workgroup's wavefronts take partitions blockIdx.x * NW + w
  // (the launch uses it only when one workgroup holds all of them) and merge
  // them in LDS; NW = 1: one partition, merged by decode_reduce_kernel.
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, j = lane >> 4;
  const int part = blockIdx.x * NW + (NW > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0);
  const int kvh = blockIdx.y, seq = blockIdx.z;
  // Clamp to what the block table can address so a bad length never reads
  // past the table.
  const int ctx = min(context_lens[seq], mbs * kBlock);
  const int tok0 = part * part_len;
  const bool empty = tok0 >= ctx;
  if (NW == 1 && empty) {
    // Empty context: the output is defined as zeros.
    if (num_parts == 1 && c < G) {
      uint16_t* orow = out + ((int64_t)seq * Hq + kvh * G + c) * D;
      for (int d = 4 * j; d < D; d += 16) *reinterpret_cast<uint64_t*>(orow + d) = 0;
    }
    return;
  }
  const int tok_end = empty ? tok0 : min(ctx, tok0 + part_len);
  const int nblk = (tok_end - tok0 + kBlock - 1) / kBlock;  // 0 for an empty partition

  const int head = kvh * G + c;
  bf16x8 qv[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (c < G)
      qv[s] = *reinterpret_cast<const bf16x8*>(q + (int64_t)seq * q_row + (int64_t)head * D + 32 * s + 8 * j);
    else
      qv[s] = bf16x8{};
  }

  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kNegBig, lsum = 0.f;

  const int32_t* btab = block_tables + (int64_t)seq * mbs + tok0 / kBlock;
  const int64_t head_stride = (int64_t)kBlock * D;  // elements per (block, head)
  constexpr int SLICE = kBlock * D * 2;  // bytes of one (block, head) of K or V
  const int koff = (c * D + 8 * j) * 2, voff = (c * kBlock + 4 * j) * 2;
  using Plain = std::integral_constant<int, 0>;
  using Stream = std::integral_constant<int, kPolicyNT>;

  // One step = two blocks (32 tokens): the K rows and Vᵀ pairs this lane
  // feeds to the MFMAs, and the blocks' valid lengths.  Steps are
  // software-pipelined two deep: the loads of step n + 1 are issued before
  // step n is computed.
  struct Step {
    bf16x8 ka[KS], kb[KS];
    uint64_t va[DT], vb[DT];
    int lim0, lim1;
  };
  auto load_step = [&](auto policy, int ib, Step& st) {
    // Block ids for this step; ids outside the pool read block 0 and are masked.
    int32_t b0 = btab[ib];
    const bool has1 = ib + 1 < nblk;
    int32_t b1 = has1 ? btab[ib + 1] : b0;
    const int rem = tok_end - (tok0 + ib * kBlock);  // tokens left from this step
    st.lim0 = rem < kBlock ? rem : kBlock;
    st.lim1 = has1 ? (rem - kBlock < kBlock ? rem - kBlock : kBlock) : 0;
    if (b0 < 0 || b0 >= num_blocks) { b0 = 0; st.lim0 = 0; }
    if (b1 < 0 || b1 >= num_blocks) { b1 = 0; st.lim1 = 0; }
    const auto rk0 = slice_rsrc(kc + ((int64_t)b0 * Hkv + kvh) * head_stride, SLICE);
    const auto rk1 = slice_rsrc(kc + ((int64_t)b1 * Hkv + kvh) * head_stride, SLICE);
    const auto rv0 = slice_rsrc(vc + ((int64_t)b0 * Hkv + kvh) * head_stride, SLICE);
    const auto rv1 = slice_rsrc(vc + ((int64_t)b1 * Hkv + kvh) * head_stride, SLICE);
    auto load_block = [&](auto policy, const __amdgpu_buffer_rsrc_t& rk,
                          const __amdgpu_buffer_rsrc_t& rv, bf16x8 (&kx)[KS],
                          uint64_t (&vx)[DT]) {
      constexpr int P = decltype(policy)::value;
#pragma unroll
      for (int s = 0; s < KS; ++s) kx[s] = __builtin_bit_cast(bf16x8, bload16<P>(rk, koff + 64 * s));
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) vx[dt] = bload8<P>(rv, voff + dt * 16 * kBlock * 2);
    };
    load_block(policy, rk0, rv0, st.ka, st.va);
    load_block(policy, rk1, rv1, st.kb, st.vb);
  };
  auto compute_step = [&](Step& st) {
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.ka[s], qv[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.kb[s], qv[s], s1, 0, 0, 0);
    }

    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s0[r] * scale_log2;
      x[4 + r] = s1[r] * scale_log2;
    }
    const int lim0 = st.lim0, lim1 = st.lim1;
    const bool partial = lim0 < kBlock || lim1 < kBlock;  // wave-uniform
    if (partial) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (4 * j + r >= lim0) x[r] = -INFINITY;
        if (4 * j + r >= lim1) x[4 + r] = -INFINITY;
      }
      // Stale cache contents beyond the context may hold any bits (NaN
      // included); zero them so 0 * V stays 0 in the P·V product.
      const int n0 = min(max(lim0 - 4 * j, 0), 4), n1 = min(max(lim1 - 4 * j, 0), 4);
      const uint64_t mk0 = n0 >= 4 ? ~0ull : ((1ull << (16 * n0)) - 1);
      const uint64_t mk1 = n1 >= 4 ? ~0ull : ((1ull << (16 * n1)) - 1);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        st.va[dt] &= mk0;
        st.vb[dt] &= mk1;
      }
    }

    float bm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                     fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    // Lazy rescale: keep the stale max unless a score exceeds it by more
    // than 2^8, so p <= 256 and the accumulator is rescaled rarely.  Lanes
    // of one head agree on m, so the exact (cross-lane) max is only needed
    // then.
    if (__builtin_amdgcn_ballot_w64(bm > m + 8.0f)) {
      bm = fmaxf(bm, shfl_xor_f(bm, 16));
      bm = fmaxf(bm, shfl_xor_f(bm, 32));
      const float mn = fmaxf(m, bm);
      const float a = fast_exp2(m - mn);
      m = mn;
      lsum *= a;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= a;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = fast_exp2(x[i] - m);
      lsum += p[i];
    }
    bf16x8 pb;
#pragma unroll
    for (int i = 0; i < 8; ++i) pb[i] = (__bf16)p[i];

#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint64_t pair[2] = {st.va[dt], st.vb[dt]};
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(pair);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
    }
  };

  // The steady-state loop issues its loads unconditionally (both steps it
  // loads exist) and with one cache policy, so the compiler's wait before a
  // step's products counts only that step's loads.  (With the next step's
  // load under a branch, or a branch between the two policies per block,
  // it waited for every load in flight, vmcnt(0), the step just issued
  // included.)  The last one or two steps run after the loop.
  auto run = [&](auto policy) {
    Step sa, sb;
    if (nblk > 0) load_step(policy, 0, sa);
    int ib = 0;
    for (; ib + 4 < nblk; ib += 4) {
      load_step(policy, ib + 2, sb);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before the products
      compute_step(sa);
      load_step(policy, ib + 4, sa);
      __builtin_amdgcn_sched_barrier(0);
      compute_step(sb);
    }
    if (ib < nblk) {
      if (ib + 2 < nblk) {
        load_step(policy, ib + 2, sb);
        __builtin_amdgcn_sched_barrier(0);
        compute_step(sa);
        compute_step(sb);
      } else {
        compute_step(sa);
      }
    }
  };
  // One policy per partition: the default (cached) one when its first block
  // is one a neighbouring sequence's table holds at the same index (a shared
  // prefix, whose blocks the other sequences then find in the cache), else
  // non-temporal.
  if (nblk > 0 && !private_block(block_tables, mbs, seq, gridDim.z, tok0 / kBlock, btab[0]))
    run(Plain{});
  else
    run(Stream{});

  lsum += shfl_xor_f(lsum, 16);
  lsum += shfl_xor_f(lsum, 32);
  if constexpr (NW > 1) {
    merge_in_workgroup<D, NW>(out + ((int64_t)seq * Hq + kvh * G) * D, o, m, lsum, c, j, G);
    return;
  }
  if (c >= G) return;
  if (num_parts == 1) {
    const float inv = lsum != 0.f ? 1.f / lsum : 0.f;
    uint16_t* orow = out + ((int64_t)seq * Hq + head) * D + 4 * j;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint16_t w[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = f32_to_bf16_bits(o[dt][r] * inv);
      *reinterpret_cast<uint64_t*>(orow + 16 * dt) = *reinterpret_cast<const uint64_t*>(w);
    }
  } else {
    const int64_t row = ((int64_t)seq * Hq + head) * num_parts + part;
    float* orow = ws_o + row * D + 4 * j;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(orow + 16 * dt) = o[dt];
    if (j == 0) {
      ws_ml[2 * row] = m;
      ws_ml[2 * row + 1] = lsum;
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA decode over FP8 caches (the reference's E4M3 codes, one byte per
// element), q / out bf16.  Same work split, online softmax and epilogue as
// decode_mfma_kernel; the operands are converted to bf16 in registers with
// v_cvt_scalef32_pk_bf16_fp8 (scale 1), except for the rare 8-byte groups
// that hold a code the OCP reading gets wrong for the reference, which take
// an exact integer decode (fp8x8_to_bf16): every code, NaN (0x80) and +-inf
// (0x7C / 0xFC) included, enters the MFMAs as the reference's value, and
// NaN / inf propagate through the scores, the softmax and P·V as IEEE
// arithmetic does in the reference.
//
// The lane layout is chosen so that every load is contiguous:
//  * QK step s: lane (c, j) supplies K rows of tokens
//      tk0 = 8 ((c >> 2) & 1) + (c & 3)  and  tk0 + 4   of block c >> 3
//    (first / second MFMA), dims D/4 j + 8 s .. + 7 (the lane's D/4 bytes of
//    each row are contiguous; Q is loaded in the same dim order).  The
//    scores then land so that lane (c, j) holds the 8 consecutive tokens
//    8 (j & 1) .. + 7 of block j >> 1.
//  * P·V: reduction slot 8 j + i is token 8 (j & 1) + i of block j >> 1, so
//    the Vᵀ operand of dims 16 dt + c is one 8-byte load from the
//    token-minor block.
// One partition of decode_fp8_kernel: where its blocks are, how a step (two
// blocks) is loaded and how it enters the online softmax.  Shared by the
// kernel's streaming loop and by fp8_exact_pass.
template <int D>
struct Fp8Partition {
  static constexpr int KS = D / 32;  // QK reduction steps
  static constexpr int DT = D / 16;  // PV output tiles
  static constexpr int DL = D / 4;   // dims (bytes) of a K row per lane group
  const uint8_t* kc;
  const uint8_t* vc;
  const int32_t* btab;  // the partition's first block-table entry
  int Hkv, kvh, num_blocks, tok0, tok_end, nblk, c, j;
  float scale_log2;
  const uint8_t* flags;  // per-block exotic-code flags (pa_decode_fp8_flagged), or null

  // The online-softmax state of a lane.
  struct State {
    f32x4 o[DT];
    float m, lsum;
  };
  // One step = two blocks; its raw K/V bytes and the blocks' valid lengths.
  struct Step {
    u32x4 k0[KS / 2], k1[KS / 2];  // 16 bytes = two reduction steps, token tk0 / tk0 + 4
    uint64_t v[DT];
    int lim0, lim1;
    uint32_t f;  // the two blocks' flags (flagged launches)
  };

  __device__ void init(State& s) const {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) s.o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    s.m = kNegBig;
    s.lsum = 0.f;
  }
  // Block ids through the scalar cache with a wait on the scalar counter only.
  // (Written out because the register-only asm elsewhere keeps the compiler
  // from proving the table unmodified; it would then read it with vector
  // loads, each followed by vmcnt(0), draining the K/V loads in flight.)
  // (Both operands are wavefront-uniform; the lane reads make that visible
  // where they arrive in vector registers, as in fp8_exact_pass.)
  __device__ int32_t table_id(int idx) const {
    const uint64_t bt = (uint64_t)(uintptr_t)btab;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)bt);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(bt >> 32));
    const int32_t* tab = (const int32_t*)(((uint64_t)hi << 32) | lo);
    int32_t v;
    asm volatile("s_load_dword %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                 : "=s"(v)
                 : "s"(tab), "s"(__builtin_amdgcn_readfirstlane(idx * 4)));
    return v;
  }
  template <bool FLAGGED = false>
  __device__ void load_step(int ib, Step& st) const {
    const int64_t head_stride = (int64_t)kBlock * D;  // bytes per (block, head)
    const bool k_second = (c >> 3) != 0;              // this lane's K rows are in block 1
    const int tk0 = 8 * ((c >> 2) & 1) + (c & 3);
    const bool v_second = (j >> 1) != 0;              // this lane's P·V tokens are in block 1
    const int tv0 = 8 * (j & 1);
    int32_t b0 = table_id(ib);
    const bool has1 = ib + 1 < nblk;
    int32_t b1 = table_id(has1 ? ib + 1 : ib);
    const int rem = tok_end - (tok0 + ib * kBlock);
    st.lim0 = rem < kBlock ? rem : kBlock;
    st.lim1 = has1 ? (rem - kBlock < kBlock ? rem - kBlock : kBlock) : 0;
    if (b0 < 0 || b0 >= num_blocks) { b0 = 0; st.lim0 = 0; }
    if (b1 < 0 || b1 >= num_blocks) { b1 = 0; st.lim1 = 0; }
    const uint8_t* kr =
        kc + ((int64_t)(k_second ? b1 : b0) * Hkv + kvh) * head_stride + tk0 * D + DL * j;
    const uint8_t* vr =
        vc + ((int64_t)(v_second ? b1 : b0) * Hkv + kvh) * head_stride + c * kBlock + tv0;
    // Non-temporal, unconditionally: a branch between load kinds makes the
    // compiler's wait counts conservative (vmcnt(0) before the first use),
    // which drains the pipeline.
#pragma unroll
    for (int s = 0; s < KS / 2; ++s) {
      st.k0[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kr + 16 * s));
      st.k1[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kr + 4 * D + 16 * s));
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      st.v[dt] = __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(vr + dt * 16 * kBlock));
    // the blocks' flag bytes arrive with the step's K / V (no round trip of
    // their own); an id outside the pool reads block 0's flag (at worst a
    // needless exact pass)
    if constexpr (FLAGGED) st.f = (uint32_t)flags[b0] | (uint32_t)flags[b1];
  }
  template <bool EXACT>
  __device__ void compute_step(Step& st, const bf16x8 (&qv)[KS], State& S) const {
    auto cvt = [](uint32_t lo, uint32_t hi) {
      return EXACT ? fp8x8_to_bf16_exact(lo, hi) : fp8x8_to_bf16(lo, hi);
    };
    const bool v_second = (j >> 1) != 0;
    const int tv0 = 8 * (j & 1);
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4& w0 = st.k0[s / 2];
      const u32x4& w1 = st.k1[s / 2];
      const int h = 2 * (s & 1);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cvt(w0[h], w0[h + 1]), qv[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cvt(w1[h], w1[h + 1]), qv[s], s1, 0, 0, 0);
    }
    // x[i] <-> token tv0 + i of this lane's block (s0: i < 4, s1: i >= 4)
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s0[r] * scale_log2;
      x[4 + r] = s1[r] * scale_log2;
    }
    if (st.lim0 < kBlock || st.lim1 < kBlock) {  // wave-uniform
      const int lim = v_second ? st.lim1 : st.lim0;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (tv0 + i >= lim) x[i] = -INFINITY;
      // Stale codes past the context may be anything; zero them so the
      // P·V product only sees zeros there.
      const int n = min(max(lim - tv0, 0), 8);
      const uint64_t mk = n >= 8 ? ~0ull : ((1ull << (8 * n)) - 1);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) st.v[dt] &= mk;
    }

    float bm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                     fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    if (__builtin_amdgcn_ballot_w64(bm > S.m + 8.0f)) {
      bm = fmaxf(bm, shfl_xor_f(bm, 16));
      bm = fmaxf(bm, shfl_xor_f(bm, 32));
      const float mn = fmaxf(S.m, bm);
      const float a = fast_exp2(S.m - mn);
      S.m = mn;
      S.lsum *= a;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) S.o[dt] *= a;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = fast_exp2(x[i] - S.m);
      S.lsum += p[i];
    }
    bf16x8 pb;
#pragma unroll
    for (int i = 0; i < 8; ++i) pb[i] = (__bf16)p[i];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      S.o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          cvt((uint32_t)st.v[dt], (uint32_t)(st.v[dt] >> 32)), pb, S.o[dt], 0, 0, 0);
  }
};

// The partition once more with the reference's exact decode of every code,
// for the rare wavefront whose streaming pass met a code the hardware
// conversion reads differently.  A call, not inlined: its registers are its
// own, so the streaming loop keeps the budget of four wavefronts per SIMD
// (the values live across the call are saved to scratch, once).
template <int D>
__device__ __attribute__((noinline)) typename Fp8Partition<D>::State fp8_exact_pass(
    const Fp8Partition<D> p, const uint16_t* qrow) {
  constexpr int KS = Fp8Partition<D>::KS;
  bf16x8 qv[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qv[s] = qrow ? *reinterpret_cast<const bf16x8*>(qrow + Fp8Partition<D>::DL * p.j + 8 * s)
                 : bf16x8{};
  typename Fp8Partition<D>::State S;
  p.init(S);
  typename Fp8Partition<D>::Step st;
  const int nblk = __builtin_amdgcn_readfirstlane(p.nblk);
  for (int ib = 0; ib < nblk; ib += 2) {
    p.load_step(ib, st);
    p.template compute_step<true>(st, qv, S);
  }
  return S;
}

// FLAGGED: the caller keeps per-block flags of the blocks that hold such
// codes (block_flags, written by pa_reshape_and_cache_fp8_flagged); the
// streaming loop then tests no codes, it ORs the step's two flag bytes, and
// a wavefront that read a flagged block takes the exact pass.  (Measured on
// the config-2 shape: 85.5 us against 88.9 us with the per-code test; with
// the test gone, two to four steps in flight at two or three wavefronts per
// SIMD, 512- or 1024-token partitions: 89.7-94.6 us; again with every load
// of the steady state unconditional and a scheduling barrier after each
// step's loads, so that each wait counted only its own step: 87.5-92.5
// against 86.7-87.0 us, partitions of 512-2048 tokens.)
template <int D, int NW, bool FLAGGED>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 4 : 1))) void decode_fp8_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q, const uint8_t* __restrict__ kc,
    const uint8_t* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ context_lens, int Hq, int Hkv, int G, int num_blocks,
    float scale_log2, int num_parts, int part_len, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, int64_t q_row, const uint8_t* __restrict__ block_flags) {
  using Part = Fp8Partition<D>;
  constexpr int KS = Part::KS;
  constexpr int DT = Part::DT;
  constexpr int DL = Part::DL;
  // NW > 1: the workgroup's wavefronts take partitions blockIdx.x * NW + w
  // (the launch uses it only when one workgroup holds all of them) and merge
  // them in LDS; NW = 1: one partition, merged by decode_reduce_kernel.
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, j = lane >> 4;
  const int part = blockIdx.x * NW + (NW > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0);
  const int kvh = blockIdx.y, seq = blockIdx.z;
  const int ctx = min(context_lens[seq], mbs * kBlock);
  const int tok0 = part * part_len;
  const bool empty = tok0 >= ctx;
  if (NW == 1 && empty) {
    if (num_parts == 1 && c < G) {
      uint16_t* orow = out + ((int64_t)seq * Hq + kvh * G + c) * D;
      for (int d = 4 * j; d < D; d += 16) *reinterpret_cast<uint64_t*>(orow + d) = 0;
    }
    return;
  }
  const int tok_end = empty ? tok0 : min(ctx, tok0 + part_len);
  const Part P{kc, vc, block_tables + (int64_t)seq * mbs + tok0 / kBlock, Hkv, kvh, num_blocks,
               tok0, tok_end, (tok_end - tok0 + kBlock - 1) / kBlock /* 0 when empty */, c, j,
               scale_log2, block_flags};

  const int head = kvh * G + c;
  const uint16_t* qrow = c < G ? q + (int64_t)seq * q_row + (int64_t)head * D : nullptr;
  bf16x8 qv[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qv[s] = qrow ? *reinterpret_cast<const bf16x8*>(qrow + DL * j + 8 * s) : bf16x8{};
  typename Part::State S;
  P.init(S);

  // Codes the hardware conversion reads differently from the reference
  // (NaN / inf / off-OCP codes; never produced from finite input) are
  // tracked per lane while the partition streams; a wavefront that met any
  // streams its partition again with the exact integer decode
  // (fp8_exact_pass: rare, and a call, so that this loop's registers stay
  // those of the plain conversion).
  uint32_t exotic = 0;
  // The q loads complete here, once: a wait for them that the compiler placed
  // inside the loop would be vmcnt(0) on every iteration and drain the
  // loads in flight.
#pragma unroll
  for (int s = 0; s < KS; ++s) asm volatile("" ::"v"(qv[s]));
  // One step in flight per wavefront and four wavefronts per SIMD (the
  // launch's partitions fill them): two steps in flight at two wavefronts
  // per SIMD measured slower, their extra VALU work less hidden.
  typename Part::Step st;
  for (int ib = 0; ib < P.nblk; ib += 2) {
    P.template load_step<FLAGGED>(ib, st);
    if constexpr (FLAGGED) {
      exotic |= st.f << 7;
    } else {
#pragma unroll
      for (int s = 0; s < KS / 2; ++s)
#pragma unroll
        for (int h = 0; h < 4; ++h)
          exotic |= fp8_exotic_bits(st.k0[s][h]) | fp8_exotic_bits(st.k1[s][h]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        exotic |= fp8_exotic_bits((uint32_t)st.v[dt]) | fp8_exotic_bits((uint32_t)(st.v[dt] >> 32));
    }
    P.template compute_step<false>(st, qv, S);
  }
  if (__builtin_amdgcn_ballot_w64((exotic & 0x80808080u) != 0)) S = fp8_exact_pass<D>(P, qrow);

  float lsum = S.lsum;
  lsum += shfl_xor_f(lsum, 16);
  lsum += shfl_xor_f(lsum, 32);
  if constexpr (NW > 1) {
    merge_in_workgroup<D, NW>(out + ((int64_t)seq * Hq + kvh * G) * D, S.o, S.m, lsum, c, j, G);
    return;
  }
  if (c >= G) return;
  if (num_parts == 1) {
    const float inv = lsum != 0.f ? 1.f / lsum : 0.f;
    uint16_t* orow = out + ((int64_t)seq * Hq + head) * D + 4 * j;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint16_t w[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = f32_to_bf16_bits(S.o[dt][r] * inv);
      *reinterpret_cast<uint64_t*>(orow + 16 * dt) = *reinterpret_cast<const uint64_t*>(w);
    }
  } else {
    const int64_t row = ((int64_t)seq * Hq + head) * num_parts + part;
    float* orow = ws_o + row * D + 4 * j;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(orow + 16 * dt) = S.o[dt];
    if (j == 0) {
      ws_ml[2 * row] = S.m;
      ws_ml[2 * row + 1] = lsum;
    }
  }
}

// ---------------------------------------------------------------------------
// Generic decode kernel: one workgroup of 256 threads per (partition, query
// head, sequence).  Scores go through LDS; f32 accumulation throughout.
template <typename T, typename TC = T>
__global__ __launch_bounds__(256) void decode_generic_kernel(
    T* __restrict__ out, const T* __restrict__ q, const TC* __restrict__ kc,
    const TC* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ context_lens, int Hq, int Hkv, int D, int num_blocks,
    float scale_log2, int num_parts, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    const float* __restrict__ kv_scales, int64_t q_row) {
  // kv_scales: per-block scales of a quantised (int8-in-f32) cache, or null
  __shared__ float qs[512];
  __shared__ float ps[kPart];
  __shared__ int32_t bs[kPart / kBlock];
  __shared__ float red[256];
  const int part = blockIdx.x, h = blockIdx.y, seq = blockIdx.z;
  const int G = Hq / Hkv, kvh = h / G;
  // Clamp to what the block table can address so a bad length never reads
  // past the table.
  const int ctx = min(context_lens[seq], mbs * kBlock);
  const int tok0 = part * kPart;
  if (tok0 >= ctx) {
    if (num_parts == 1)
      for (int d = threadIdx.x; d < D; d += blockDim.x)
        Elem<T>::store(out + ((int64_t)seq * Hq + h) * D + d, 0.f);
    return;
  }
  const int n = min(ctx - tok0, kPart);
  const int tid = threadIdx.x;
  for (int d = tid; d < D; d += blockDim.x)
    qs[d] = Elem<T>::load(q + (int64_t)seq * q_row + (int64_t)h * D + d);
  if (tid < (n + kBlock - 1) / kBlock) {
    const int32_t b = block_tables[(int64_t)seq * mbs + tok0 / kBlock + tid];
    bs[tid] = (b >= 0 && b < num_blocks) ? b : -1;
  }
  __syncthreads();

  float mloc = -INFINITY;
  for (int t = tid; t < n; t += blockDim.x) {
    const int32_t b = bs[t / kBlock];
    float s = -INFINITY;
    if (b >= 0) {
      const TC* kr = kc + (((int64_t)b * Hkv + kvh) * kBlock + t % kBlock) * D;
      const float ks = kv_scales ? kv_scales[b] : 1.0f;
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc += qs[d] * (Elem<TC>::load(kr + d) * ks);
      s = acc * scale_log2;
    }
    ps[t] = s;
    mloc = fmaxf(mloc, s);
  }
  red[tid] = mloc;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if (tid < w) red[tid] = fmaxf(red[tid], red[tid + w]);
    __syncthreads();
  }
  const float m = red[0] == -INFINITY ? kNegBig : red[0];
  __syncthreads();
  float lloc = 0.f;
  for (int t = tid; t < n; t += blockDim.x) {
    const float p = exp2f(ps[t] - m);
    ps[t] = p;
    lloc += p;
  }
  red[tid] = lloc;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  const float l = red[0];
  for (int d = tid; d < D; d += blockDim.x) {
    float acc = 0.f;
    for (int t = 0; t < n; ++t) {
      const int32_t b = bs[t / kBlock];
      if (b < 0) continue;
      const float vs = kv_scales ? kv_scales[b] : 1.0f;
      acc += ps[t] * (Elem<TC>::load(vc + (((int64_t)b * Hkv + kvh) * D + d) * kBlock + t % kBlock) * vs);
    }
    if (num_parts == 1) {
      Elem<T>::store(out + ((int64_t)seq * Hq + h) * D + d, l != 0.f ? acc / l : 0.f);
    } else {
      ws_o[(((int64_t)seq * Hq + h) * num_parts + part) * D + d] = acc;
    }
  }
  if (num_parts > 1 && tid == 0) {
    const int64_t row = ((int64_t)seq * Hq + h) * num_parts + part;
    ws_ml[2 * row] = m;
    ws_ml[2 * row + 1] = l;
  }
}

// ---------------------------------------------------------------------------
// f32 caches (plain, or int8-in-f32 with one scale per block): one workgroup
// of 4 PL threads per (partition of PL tokens, kv head, sequence) serving
// all G query heads of the group, so each K / V byte is read once for the
// group.  Small decode batches are latency-bound, so the work of a thread
// is kept short and every load is issued at the start:
//   QK:  four adjacent lanes per token, each a quarter of the K row (the
//        four read one contiguous row), partial dot products with the G
//        query rows (LDS) combined by two lane shuffles.
//   softmax: one wavefront per query head, over the partition.
//   PV:  lane (d, r) owns dim d of the blocks r, r + R, ... (R = 4 PL / D);
//        the R lanes of one dim are adjacent, so their partial sums are
//        combined by lane shuffles.
// Partial results use the split-K workspace format of decode_reduce_kernel.
constexpr int kF32MaxG = 16;
// PL = 256, or 128 for launches of few (kv head, sequence) pairs: a CU
// reads its workgroup's K / V at a bounded rate (what it keeps in flight
// over the memory latency), so small launches finish sooner spread over
// twice the workgroups (query groups of at most 8 heads: one wavefront
// each in the softmax).
template <int D, int PL>
__global__ __launch_bounds__(4 * PL) void decode_f32_group_kernel(
    float* __restrict__ out, const float* __restrict__ q, const float* __restrict__ kc,
    const float* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ context_lens, int Hq, int Hkv, int num_blocks,
    float scale_log2, int num_parts, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    const float* __restrict__ kv_scales, int64_t q_row) {
  static_assert(256 % D == 0 && D % 16 == 0, "head_dim must divide 256, in 16-float steps");
  constexpr int NTH = 4 * PL;                // threads
  constexpr int NPB = PL / kBlock;           // blocks per partition
  constexpr int R = NTH / D;                 // lanes per dim in P·V (a power of two <= 64)
  static_assert(R >= 1 && R <= 64, "lanes per dim");
  constexpr int NBT = NPB >= R ? NPB / R : 1;  // blocks per lane in P·V
  constexpr int KQ = D / 16;                 // float4 per lane of a K row quarter
  __shared__ __attribute__((aligned(16))) float qs[kF32MaxG * D];
  __shared__ __attribute__((aligned(16))) float ps[kF32MaxG][PL];
  __shared__ int32_t bs[NPB];
  __shared__ float bsc[NPB];
  __shared__ float mls[kF32MaxG][2];
  const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int G = Hq / Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The block ids and the query rows are loaded in the same round trip as
  // the context length (they depend only on the partition's position).
  const int tok0 = part * PL;
  const int bi0 = tok0 / kBlock;
  int32_t braw = -1;
  if (tid < NPB && bi0 + tid < mbs) braw = block_tables[(int64_t)seq * mbs + bi0 + tid];
  for (int e = tid; e < G * D; e += NTH) qs[e] = q[(int64_t)seq * q_row + (int64_t)kvh * G * D + e];
  const int ctx = min(context_lens[seq], mbs * kBlock);
  if (tok0 >= ctx) {
    if (num_parts == 1)
      for (int e = tid; e < G * D; e += NTH) out[((int64_t)seq * Hq + kvh * G) * D + e] = 0.f;
    return;
  }
  const int n = min(ctx - tok0, PL);
  const int nb = (n + kBlock - 1) / kBlock;
  if (tid < NPB) {
    const bool ok = tid < nb && braw >= 0 && braw < num_blocks;
    bs[tid] = ok ? braw : -1;
    bsc[tid] = ok && kv_scales ? kv_scales[braw] : 1.0f;
  }
  __syncthreads();

  // V rows of this lane's P·V share, loaded before anything else needs them
  const int d = wave * (64 / R) + lane / R, r = lane % R;
  float4 vx[NBT][4];
#pragma unroll
  for (int i = 0; i < NBT; ++i) {
    const int bi = r + i * R;
    const int32_t b = bi < nb ? bs[bi] : -1;
    const float* vr = vc + (((int64_t)(b >= 0 ? b : 0) * Hkv + kvh) * D + d) * kBlock;
#pragma unroll
    for (int x = 0; x < 4; ++x)
      vx[i][x] = b >= 0 ? *reinterpret_cast<const float4*>(vr + 4 * x) : float4{0.f, 0.f, 0.f, 0.f};
  }

  // QK: token t, quarter qq of its row
  {
    const int t = tid >> 2, qq = tid & 3;
    const int32_t b = t < n ? bs[t / kBlock] : -1;
    const float* kr = kc + (((int64_t)(b >= 0 ? b : 0) * Hkv + kvh) * kBlock + t % kBlock) * D +
                      qq * (D / 4);
    float4 kx[KQ];
#pragma unroll
    for (int i = 0; i < KQ; ++i)
      kx[i] = b >= 0 ? *reinterpret_cast<const float4*>(kr + 4 * i) : float4{0.f, 0.f, 0.f, 0.f};
    const float ks = b >= 0 ? bsc[t / kBlock] * scale_log2 : 0.f;
    for (int g = 0; g < G; ++g) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < KQ; ++i) {
        const float4 qx = *reinterpret_cast<const float4*>(&qs[g * D + qq * (D / 4) + 4 * i]);
        acc += qx.x * kx[i].x + qx.y * kx[i].y + qx.z * kx[i].z + qx.w * kx[i].w;
      }
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      if (qq == 0) ps[g][t] = b >= 0 ? acc * ks : -INFINITY;
    }
  }
  __syncthreads();

  // softmax over the partition, one wavefront per query head
  if (wave < G) {
    const int g = wave;
    float v[PL / 64];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL / 64; ++i) {
      v[i] = ps[g][lane + 64 * i];
      mx = fmaxf(mx, v[i]);
    }
    for (int w = 32; w > 0; w >>= 1) mx = fmaxf(mx, __shfl_xor(mx, w, 64));
    const float m = mx == -INFINITY ? kNegBig : mx;
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < PL / 64; ++i) {
      const float p = exp2f(v[i] - m);
      ps[g][lane + 64 * i] = p;
      l += p;
    }
    for (int w = 32; w > 0; w >>= 1) l += __shfl_xor(l, w, 64);
    if (lane == 0) {
      mls[g][0] = m;
      mls[g][1] = l;
    }
  }
  __syncthreads();

  // PV: lane (d, r) over the blocks r, r + R, ..., then the R lanes of dim d
  // combined; lane r == 0 writes
  for (int g = 0; g < G; ++g) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NBT; ++i) {
      const int bi = r + i * R;
      if (bi < nb) {
        const float* pg = &ps[g][bi * kBlock];
        float a = 0.f;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const float4 px = *reinterpret_cast<const float4*>(pg + 4 * x);
          a += px.x * vx[i][x].x + px.y * vx[i][x].y + px.z * vx[i][x].z + px.w * vx[i][x].w;
        }
        acc += a * bsc[bi];
      }
    }
#pragma unroll
    for (int w = 1; w < R; w <<= 1) acc += __shfl_xor(acc, w, 64);
    if (r == 0) {
      const int64_t row = (int64_t)seq * Hq + kvh * G + g;
      if (num_parts == 1) {
        const float l = mls[g][1];
        out[row * D + d] = l != 0.f ? acc / l : 0.f;
      } else {
        ws_o[(row * num_parts + part) * D + d] = acc;
        if (d == 0) {
          ws_ml[2 * (row * num_parts + part)] = mls[g][0];
          ws_ml[2 * (row * num_parts + part) + 1] = mls[g][1];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Balanced split-K ("stream-K") decode for long, ragged contexts.
//
// A partitioned launch gives every (sequence, kv head) the same number of
// fixed-length partitions; with ragged contexts the workgroups of the last
// dispatch round run with the GPU mostly idle (measured on BASELINE config
// 4: about 2000 wavefronts in flight for 110 us, then a 55 us tail in which
// they drain).  Here the work is cut evenly instead: a unit is one 32-token
// step of one (sequence, kv head) segment, the segments are laid end to end
// (sequence-major, kv head minor), and wavefront w of N takes units
// [floor(w U / N), floor((w + 1) U / N)) of the U in all, crossing segment
// boundaries as it goes.  For every segment piece it writes one partial
// result (m, l, o per query head) into slot w - first(segment) of the
// segment's rows; decode_reduce_kernel merges a row's slots.  Both kernels
// derive U, N and a segment's first and last wavefront from context_lens
// the same way, so no offsets travel between them.
// Measured on config 4 (B 16, contexts 8k-32k, flushed caches): 162 us
// against 177 us for 512-token partitions; with every block private, 6.2
// TB/s.  One wavefront per SIMD: the two-deep step pipeline takes most of
// the register file (2048 or more wavefronts of the unpipelined loop
// measured 2-20% slower).
constexpr int kBalanceMinUnits = 8;   // units per wavefront at least (256 tokens)
constexpr int kBalanceWaves = 1024;   // one wavefront per SIMD of the 256 CUs

// A wavefront-uniform 64-bit value held in vector registers, moved to
// scalar ones (every lane holds the same value).
__device__ inline int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
// Context lengths are clamped to the table and to the launch's
// max_context_len (`cap`): the workspace slots are sized from it, so a
// length above it (a caller error) never gets more slots than a row has.
__device__ inline int seq_units(const int32_t* __restrict__ context_lens, int s, int mbs,
                                int cap) {
  const int ctx = min(min(context_lens[s], mbs * kBlock), cap);
  return ctx > 0 ? (ctx + 2 * kBlock - 1) / (2 * kBlock) : 0;
}

// Work layout of a balanced launch.  Sequences are taken in groups of at
// most SP (= 16 / G, the sequences whose query heads fill the 16 MFMA
// columns together) that begin with the same block (a prefix-cache hit:
// decode_group_kernel sorts the sequences by their first block, wherever
// they sit in the batch, and cuts each run of equal first blocks into
// groups of SP).  lcp[g] is the number of leading units every member of
// group g holds in full and whose blocks all members' tables share (a
// common prefix).  Group g's units:
//   the shared segments (kv head 0 .. Hkv-1, lcp[g] units each, every
//   member attended at once), then for each member the private segments
//   (kv head 0 .. Hkv-1, its units past the prefix).
// Without sharing (grp null) every sequence is its own group, in order.
//
// The group record `grp` (int32, 6 B + 2 entries, written by
// decode_group_kernel): [0] group count ng; order[B] (sequence at each
// sorted position); gstart[B + 1] (first position of each group, gstart[ng]
// = B); gof[B] (group of each sequence); pos[B] (sorted position of each
// sequence); lcp[B] (shared units of each group); gsum[B] (the members'
// units summed, so a group's size needs no walk over its members).
constexpr int kGrpOrder = 1;
__device__ inline int grp_gstart(int B) { return 1 + B; }
__device__ inline int grp_gof(int B) { return 2 + 2 * B; }
__device__ inline int grp_pos(int B) { return 2 + 3 * B; }
__device__ inline int grp_lcp(int B) { return 2 + 4 * B; }
__device__ inline int grp_gsum(int B) { return 2 + 5 * B; }

struct BalanceLayout {
  const int32_t* __restrict__ ctx;
  const int32_t* __restrict__ grp;  // null: no shared prefixes
  int B, mbs, Hkv, cap;
  __device__ int units(int s) const { return seq_units(ctx, s, mbs, cap); }
  __device__ int groups() const { return grp ? grp[0] : B; }
  // first sorted position of group g (g <= groups())
  __device__ int first(int g) const { return grp ? grp[grp_gstart(B) + g] : g; }
  __device__ int member(int p) const { return grp ? grp[kGrpOrder + p] : p; }
  __device__ int group_of(int s) const { return grp ? grp[grp_gof(B) + s] : s; }
  __device__ int pos_of(int s) const { return grp ? grp[grp_pos(B) + s] : s; }
  __device__ int shared(int g) const { return grp ? grp[grp_lcp(B) + g] : 0; }
  __device__ int64_t group_units(int g) const {
    if (!grp) return (int64_t)units(g) * Hkv;
    const int L = shared(g), gn = first(g + 1) - first(g);
    return ((int64_t)L + grp[grp_gsum(B) + g] - (int64_t)gn * L) * Hkv;
  }
  // units of the groups before `upto`, summed over a wavefront (every lane
  // returns the same value)
  __device__ int64_t before(int upto) const {
    const int lane = threadIdx.x & 63;
    int64_t acc = 0;
    for (int g = lane; g < upto; g += 64) acc += group_units(g);
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    return uniform64(acc);
  }
};
__device__ inline int balance_waves(int64_t total, int max_waves) {
  return (int)max((int64_t)1, min((int64_t)max_waves, total / kBalanceMinUnits));
}
// The wavefront whose range holds unit g: the largest w with
// floor(w U / N) <= g.
__device__ inline int wave_of(int64_t g, int64_t total, int nw) {
  return (int)(((g + 1) * nw - 1) / total);
}
// Slots of a segment [start, start + len): its first to its last wavefront.
// Every wavefront's range holds at least kBalanceMinUnits units (N <= U /
// kBalanceMinUnits), so a segment of n units meets at most
// floor((n - 2) / kBalanceMinUnits) + 2 <= ceil(n / kBalanceMinUnits) + 1
// wavefronts, and a row's two segments (n units in all) at most
// ceil(n / kBalanceMinUnits) + 3: the slots per row decode_plan sizes.
__device__ inline int seg_slots(int64_t start, int len, int64_t total, int nw) {
  return len > 0 ? wave_of(start + len - 1, total, nw) - wave_of(start, total, nw) + 1 : 0;
}

// Shared-prefix groups and their common prefixes, in full units.  Every
// workgroup (one per possible group, B in all) sorts the sequences by
// (first block id, index) in LDS, redundantly, so no second launch is
// needed: each thread ranks one key against all B <= kGroupMaxSeqs
// (broadcast LDS reads, four barriers in all; a bitonic sort's ~40
// barriers of 16 wavefronts cost 3 us more at B 16), cuts the runs of
// sequences that begin with the same block into groups of at most SP, and
// workgroup g finds group g's common
// prefix: every table entry a member may share is loaded and compared at
// once, and the first differing block is the workgroup's minimum.
// Workgroup 0 writes the group record.  A sequence holding no full unit
// (32 tokens) shares nothing and is a group of its own.
constexpr int kGroupThreads = 1024;
constexpr int kGroupMaxSeqs = 1024;  // larger launches are not grouped
__global__ __launch_bounds__(kGroupThreads) void decode_group_kernel(
    const int32_t* __restrict__ block_tables, int mbs, const int32_t* __restrict__ context_lens,
    int B, int SP, int cap, int32_t* __restrict__ grp) {
  __shared__ uint64_t raw[kGroupMaxSeqs];
  __shared__ uint64_t key[kGroupMaxSeqs];   // sorted
  __shared__ uint8_t newg[kGroupMaxSeqs];   // a group starts at this position
  __shared__ int32_t gid[kGroupMaxSeqs];
  __shared__ int32_t gst[kGroupMaxSeqs + 1];
  __shared__ int first_diff;
  const int tid = threadIdx.x, g = blockIdx.x;
  constexpr uint32_t kNone = 0xFFFFFFFFu;  // first "block" of a sequence that shares nothing
  if (tid < B) {
    const int units = min(min(context_lens[tid], mbs * kBlock), cap) / (2 * kBlock);
    const uint32_t id = units > 0 ? (uint32_t)block_tables[(int64_t)tid * mbs] : kNone;
    raw[tid] = ((uint64_t)id << 32) | (uint32_t)tid;
  }
  if (tid == 0) first_diff = INT32_MAX;
  __syncthreads();
  if (tid < B) {  // the keys are distinct (the index is in the low half)
    const uint64_t k = raw[tid];
    int rank = 0;
    for (int t = 0; t < B; ++t) rank += raw[t] < k;
    key[rank] = k;
  }
  __syncthreads();
  // runs of equal first blocks (a sequence that shares nothing is a run of
  // its own), cut into groups of SP
  if (tid < B) {
    const uint32_t hi = (uint32_t)(key[tid] >> 32);
    int r0 = tid;
    if (hi != kNone)
      while (r0 > 0 && (uint32_t)(key[r0 - 1] >> 32) == hi) --r0;
    newg[tid] = (tid - r0) % SP == 0;
  }
  __syncthreads();
  if (tid < B) {
    int n = 0;
    for (int t = 0; t <= tid; ++t) n += newg[t];
    gid[tid] = n - 1;
    if (newg[tid]) gst[n - 1] = tid;
  }
  __syncthreads();
  const int ng = gid[B - 1] + 1;
  if (tid == 0) gst[ng] = B;
  __syncthreads();
  if (g == 0) {
    if (tid == 0) grp[0] = ng;
    for (int r = tid; r < B; r += kGroupThreads) {
      const int s = (int)(uint32_t)key[r];
      grp[kGrpOrder + r] = s;
      grp[grp_gof(B) + s] = gid[r];
      grp[grp_pos(B) + s] = r;
    }
    for (int r = tid; r <= ng; r += kGroupThreads) grp[grp_gstart(B) + r] = gst[r];
  }
  if (g >= ng) return;
  const int p0 = gst[g], gn = gst[g + 1] - p0;
  const int s0 = (int)(uint32_t)key[p0];
  int L = INT32_MAX;
  for (int m = 0; m < gn; ++m) {
    const int s = (int)(uint32_t)key[p0 + m];
    L = min(L, min(min(context_lens[s], mbs * kBlock), cap) / (2 * kBlock));
  }
  // a member's negative length (a caller error) shares nothing: L >= 0
  if (gn < 2 || L < 0) L = 0;
  // blocks below 2 L where a member's table differs from the first's (the
  // loads do not wait for L: every index below mbs is inside the tables)
  int diff = INT32_MAX;
  for (int b = tid; b < mbs; b += kGroupThreads) {
    const int32_t id = block_tables[(int64_t)s0 * mbs + b];
    bool d = false;
    for (int m = 1; m < gn; ++m)
      d |= block_tables[(int64_t)(uint32_t)key[p0 + m] * mbs + b] != id;
    if (d && b < 2 * L) diff = min(diff, b);
  }
  for (int o = 32; o > 0; o >>= 1) diff = min(diff, __shfl_xor(diff, o, 64));
  if ((tid & 63) == 0 && diff != INT32_MAX) atomicMin(&first_diff, diff);
  __syncthreads();
  if (tid == 0) {
    grp[grp_lcp(B) + g] = min(L, first_diff / 2);
    int sum = 0;
    for (int m = 0; m < gn; ++m) sum += seq_units(context_lens, (int)(uint32_t)key[p0 + m], mbs, cap);
    grp[grp_gsum(B) + g] = sum;
  }
}

// One segment piece: kv head kvh, units [u0, u1) of the segment.  Shared
// pieces attend group members [g0, g0 + gn) at once (MFMA column c: member
// c / G, head c % G; every member holds the units in full, the blocks from
// the first member's table); private pieces one sequence (column c: head
// c), its units past the shared prefix.
struct Piece {
  bool shared;
  int seq;      // private: the sequence; shared: the group's first member
  int p0, gn;   // shared: the group's first sorted position, members
  int kvh, u0, u1, unit_base;  // unit_base: the segment's first unit within the sequence
  int64_t start;  // the segment's first unit in the layout
  int slot_base;  // private: the row's shared slots
};

template <int D>
__global__ __launch_bounds__(64) void decode_balanced_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ context_lens, int B, int Hq, int Hkv, int G, int num_blocks,
    float scale_log2, int slots, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    int64_t q_row, const int32_t* __restrict__ grp, int cap) {
  constexpr int KS = D / 32;  // QK reduction steps
  constexpr int DT = D / 16;  // PV output tiles
  const int lane = threadIdx.x;
  const int c = lane & 15, j = lane >> 4;
  const BalanceLayout lay{context_lens, grp, B, mbs, Hkv, cap};
  const int64_t total = lay.before(lay.groups());
  const int nw = balance_waves(total, gridDim.x);
  const int w = blockIdx.x;
  if (total == 0 || w >= nw) return;
  const int64_t lo = (int64_t)w * total / nw, hi = (int64_t)(w + 1) * total / nw;
  if (lo >= hi) return;

  // The group holding unit lo: scan the per-group unit counts 64 at a time
  // (inclusive prefix sums across the wavefront).
  const int ng = lay.groups();
  int g = 0;
  int64_t cg = 0;  // first unit of group g
  for (int base = 0; base < ng; base += 64) {
    const int64_t n = base + lane < ng ? lay.group_units(base + lane) : 0;
    int64_t incl = n;
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t t = __shfl_up(incl, o, 64);
      if (lane >= o) incl += t;
    }
    const uint64_t past = __builtin_amdgcn_ballot_w64(cg + incl > lo);
    if (past) {
      const int first = __builtin_ctzll(past);
      g = base + first;
      cg = uniform64(cg + __shfl(incl, first, 64) - __shfl(n, first, 64));
      break;
    }
    cg = uniform64(cg + __shfl(incl, 63, 64));
  }

  const int64_t head_stride = (int64_t)kBlock * D;
  constexpr int SLICE = kBlock * D * 2;
  const int koff = (c * D + 8 * j) * 2, voff = (c * kBlock + 4 * j) * 2;
  struct Step {
    bf16x8 ka[KS], kb[KS];
    uint64_t va[DT], vb[DT];
    int lim0, lim1;
  };
  for (int64_t gpos = lo; gpos < hi && g < ng;) {
    const int64_t gu = lay.group_units(g);
    if (gpos >= cg + gu) {  // next group
      cg += gu;
      ++g;
      continue;
    }
    // the segment holding gpos
    const int L = lay.shared(g), p0 = lay.first(g), gn = lay.first(g + 1) - p0;
    int64_t r = gpos - cg;
    Piece pc{};
    if (r < (int64_t)Hkv * L) {
      pc.shared = true;
      pc.seq = lay.member(p0);
      pc.p0 = p0;
      pc.gn = gn;
      pc.kvh = (int)(r / L);
      pc.u0 = (int)(r % L);
      pc.u1 = L;
      pc.unit_base = 0;
      pc.start = cg + (int64_t)pc.kvh * L;
    } else {
      r -= (int64_t)Hkv * L;
      int64_t off = (int64_t)Hkv * L;
      pc.seq = -1;
      for (int mp = p0; mp < p0 + gn; ++mp) {  // gpos lies in this group: a member holds it
        const int m = lay.member(mp);
        const int len = lay.units(m) - L;
        if (len > 0 && r < (int64_t)Hkv * len) {
          pc.seq = m;
          pc.kvh = (int)(r / len);
          pc.u0 = (int)(r % len);
          pc.u1 = len;
          pc.unit_base = L;
          pc.start = cg + off + (int64_t)pc.kvh * len;
          // the row's shared slots come first
          pc.slot_base = seg_slots(cg + (int64_t)pc.kvh * L, L, total, nw);
          break;
        }
        r -= (int64_t)Hkv * max(len, 0);
        off += (int64_t)Hkv * max(len, 0);
      }
      if (pc.seq < 0) break;  // (not reached: the layout sums to gu)
    }
    pc.u1 = (int)min((int64_t)pc.u1, pc.u0 + (hi - gpos));
    const int kvh = pc.kvh;
    const int ctx = min(min(context_lens[pc.seq], mbs * kBlock), cap);
    const int tok0 = (pc.unit_base + pc.u0) * 2 * kBlock;
    const int tok_end = pc.shared ? (pc.unit_base + pc.u1) * 2 * kBlock
                                  : min(ctx, (pc.unit_base + pc.u1) * 2 * kBlock);
    const int nblk = (tok_end - tok0 + kBlock - 1) / kBlock;
    // this lane's MFMA column: sequence and query head
    const bool col_ok = pc.shared ? c < pc.gn * G : c < G;
    const int col_seq = pc.shared ? (col_ok ? lay.member(pc.p0 + c / G) : pc.seq) : pc.seq;
    const int head = kvh * G + (pc.shared ? c % G : c);
    bf16x8 qv[KS];
#pragma unroll
    for (int st = 0; st < KS; ++st)
      qv[st] = col_ok ? *reinterpret_cast<const bf16x8*>(q + (int64_t)col_seq * q_row +
                                                         (int64_t)head * D + 32 * st + 8 * j)
                      : bf16x8{};
    f32x4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = kNegBig, lsum = 0.f;
    const int32_t* btab = block_tables + (int64_t)pc.seq * mbs + tok0 / kBlock;
    // Steps software-pipelined two deep for D <= 128, as decode_mfma_kernel:
    // the loads are unconditional non-temporal loads and the block ids come
    // through explicit scalar loads, so the compiler's wait counts stay
    // exact.
    auto table_id = [&](int idx) -> int32_t {
      int32_t v;
      asm volatile("s_load_dword %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                   : "=s"(v)
                   : "s"(btab), "s"(idx * 4));
      return v;
    };
    auto load_step = [&](int ib, Step& st) {
      int32_t b0 = table_id(ib);
      const bool has1 = ib + 1 < nblk;
      int32_t b1 = table_id(has1 ? ib + 1 : ib);
      const int rem = tok_end - (tok0 + ib * kBlock);
      st.lim0 = rem < kBlock ? rem : kBlock;
      st.lim1 = has1 ? (rem - kBlock < kBlock ? rem - kBlock : kBlock) : 0;
      if (b0 < 0 || b0 >= num_blocks) { b0 = 0; st.lim0 = 0; }
      if (b1 < 0 || b1 >= num_blocks) { b1 = 0; st.lim1 = 0; }
      const auto rk0 = slice_rsrc(kc + ((int64_t)b0 * Hkv + kvh) * head_stride, SLICE);
      const auto rk1 = slice_rsrc(kc + ((int64_t)b1 * Hkv + kvh) * head_stride, SLICE);
      const auto rv0 = slice_rsrc(vc + ((int64_t)b0 * Hkv + kvh) * head_stride, SLICE);
      const auto rv1 = slice_rsrc(vc + ((int64_t)b1 * Hkv + kvh) * head_stride, SLICE);
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        st.ka[t] = __builtin_bit_cast(bf16x8, bload16<kPolicyNT>(rk0, koff + 64 * t));
        st.kb[t] = __builtin_bit_cast(bf16x8, bload16<kPolicyNT>(rk1, koff + 64 * t));
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        st.va[dt] = bload8<kPolicyNT>(rv0, voff + dt * 16 * kBlock * 2);
        st.vb[dt] = bload8<kPolicyNT>(rv1, voff + dt * 16 * kBlock * 2);
      }
    };
    auto compute = [&](Step& st) {
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.ka[t], qv[t], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.kb[t], qv[t], s1, 0, 0, 0);
      }
      float x[8];
#pragma unroll
      for (int r2 = 0; r2 < 4; ++r2) {
        x[r2] = s0[r2] * scale_log2;
        x[4 + r2] = s1[r2] * scale_log2;
      }
      if (st.lim0 < kBlock || st.lim1 < kBlock) {  // wave-uniform
#pragma unroll
        for (int r2 = 0; r2 < 4; ++r2) {
          if (4 * j + r2 >= st.lim0) x[r2] = -INFINITY;
          if (4 * j + r2 >= st.lim1) x[4 + r2] = -INFINITY;
        }
        // stale cache contents beyond the context may hold any bits
        const int n0 = min(max(st.lim0 - 4 * j, 0), 4), n1 = min(max(st.lim1 - 4 * j, 0), 4);
        const uint64_t mk0 = n0 >= 4 ? ~0ull : ((1ull << (16 * n0)) - 1);
        const uint64_t mk1 = n1 >= 4 ? ~0ull : ((1ull << (16 * n1)) - 1);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          st.va[dt] &= mk0;
          st.vb[dt] &= mk1;
        }
      }
      float bm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                       fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
      if (__builtin_amdgcn_ballot_w64(bm > m + 8.0f)) {  // lazy rescale
        bm = fmaxf(bm, shfl_xor_f(bm, 16));
        bm = fmaxf(bm, shfl_xor_f(bm, 32));
        const float mn = fmaxf(m, bm);
        const float a = fast_exp2(m - mn);
        m = mn;
        lsum *= a;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= a;
      }
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = fast_exp2(x[i] - m);
        lsum += p[i];
      }
      bf16x8 pb;
#pragma unroll
      for (int i = 0; i < 8; ++i) pb[i] = (__bf16)p[i];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint64_t pair[2] = {st.va[dt], st.vb[dt]};
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(pair);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
      }
    };
#pragma unroll
    for (int st = 0; st < KS; ++st) asm volatile("" ::"v"(qv[st]));
    if constexpr (D <= 128) {
      // unconditional loads in the steady state and a scheduling barrier
      // after each step's loads, as in decode_mfma_kernel
      Step sa, sb;
      if (nblk > 0) load_step(0, sa);
      int ib = 0;
      for (; ib + 4 < nblk; ib += 4) {
        load_step(ib + 2, sb);
        __builtin_amdgcn_sched_barrier(0);
        compute(sa);
        load_step(ib + 4, sa);
        __builtin_amdgcn_sched_barrier(0);
        compute(sb);
      }
      if (ib < nblk) {
        if (ib + 2 < nblk) {
          load_step(ib + 2, sb);
          __builtin_amdgcn_sched_barrier(0);
          compute(sa);
          compute(sb);
        } else {
          compute(sa);
        }
      }
    } else {
      // D = 256: two steps do not fit the register file; one at a time
      for (int ib = 0; ib < nblk; ib += 2) {
        Step st;
        load_step(ib, st);
        compute(st);
      }
    }
    lsum += shfl_xor_f(lsum, 16);
    lsum += shfl_xor_f(lsum, 32);
    const int k = (pc.shared ? 0 : pc.slot_base) + w - wave_of(pc.start, total, nw);
    if (col_ok && k < slots) {  // (k < slots always holds: seg_slots' bound; a guard)
      const int64_t row = ((int64_t)col_seq * Hq + head) * slots + k;
      float* orow = ws_o + row * D + 4 * j;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(orow + 16 * dt) = o[dt];
      if (j == 0) {
        ws_ml[2 * row] = m;
        ws_ml[2 * row + 1] = lsum;
      }
    }
    gpos += pc.u1 - pc.u0;
  }
}

// ---------------------------------------------------------------------------
// Partition merge: one workgroup of 256 threads per (sequence, query head).
// Wavefront w merges the partitions w, w + 4, ... in chunks of kRU whose
// (m, l) pairs and output dims are loaded together (one round trip per
// chunk), keeping a running max; the four wavefronts' (M, L, o) are then
// merged through LDS with the same log-sum-exp rule.  Lane t holds dims
// t, t + 64, ... (head_dim <= 64 * kDL).
template <typename T, int kDL>
__global__ __launch_bounds__(256) void decode_reduce_kernel(
    T* __restrict__ out, const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ context_lens, int Hq, int D, int num_parts, int mbs,
    int part_len, int balance_nw, int B, int Hkv, const int32_t* __restrict__ grp, int cap) {
  // balance_nw > 0: partial results of decode_balanced_kernel launched with
  // balance_nw wavefronts (num_parts = slots per row; grp its groups);
  // else partitions of part_len tokens.
  __shared__ float red[4][64 * kDL];
  __shared__ float wml[2][4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row = blockIdx.x;  // seq * Hq + head
  const int seq = row / Hq;
  const int ctx = min(context_lens[seq], mbs * kBlock);
  int np;
  if (balance_nw > 0) {
    // this row's slots: those of its group's shared segment, then those of
    // its private segment
    const BalanceLayout lay{context_lens, grp, B, mbs, Hkv, cap};
    const int64_t total = lay.before(lay.groups());
    np = 0;
    if (total > 0) {
      const int nw = balance_waves(total, balance_nw);
      const int g = lay.group_of(seq), kvh = (row % Hq) / (Hq / Hkv);
      const int64_t cg = lay.before(g);
      const int L = lay.shared(g);
      int64_t off = cg + (int64_t)Hkv * L;
      for (int p = lay.first(g), pe = lay.pos_of(seq); p < pe; ++p)
        off += (int64_t)Hkv * (lay.units(lay.member(p)) - L);
      const int len = lay.units(seq) - L;
      // (the cap never binds: seg_slots' bound sizes num_parts; it keeps
      // the reads inside the row whatever the inputs)
      np = min(seg_slots(cg + (int64_t)kvh * L, L, total, nw) +
                   seg_slots(off + (int64_t)kvh * len, len, total, nw),
               num_parts);
    }
  } else {
    np = min(num_parts, (ctx + part_len - 1) / part_len);
  }
  const int64_t row0 = (int64_t)row * num_parts;
  constexpr int kRU = 8;
  float M = -INFINITY, L = 0.f, acc[kDL];
#pragma unroll
  for (int k = 0; k < kDL; ++k) acc[k] = 0.f;
  for (int p0 = wave; p0 < np; p0 += 4 * kRU) {
    float2 ml[kRU];
    float v[kRU][kDL];
#pragma unroll
    for (int u = 0; u < kRU; ++u) {
      const int64_t p = row0 + min(p0 + 4 * u, np - 1);
      ml[u] = float2{ws_ml[2 * p], ws_ml[2 * p + 1]};
#pragma unroll
      for (int k = 0; k < kDL; ++k) v[u][k] = lane + 64 * k < D ? ws_o[p * D + lane + 64 * k] : 0.f;
    }
    float cm = M;
#pragma unroll
    for (int u = 0; u < kRU; ++u)
      if (p0 + 4 * u < np) cm = fmaxf(cm, ml[u].x);
    if (cm == -INFINITY) continue;  // no keys so far
    const float r = exp2f(M - cm);  // 0 while M is -inf
    L *= r;
#pragma unroll
    for (int k = 0; k < kDL; ++k) acc[k] *= r;
#pragma unroll
    for (int u = 0; u < kRU; ++u) {
      if (p0 + 4 * u < np) {
        const float w = exp2f(ml[u].x - cm);
        L += w * ml[u].y;
#pragma unroll
        for (int k = 0; k < kDL; ++k) acc[k] += w * v[u][k];
      }
    }
    M = cm;
  }
#pragma unroll
  for (int k = 0; k < kDL; ++k)
    if (lane + 64 * k < D) red[wave][lane + 64 * k] = acc[k];
  if (lane == 0) {
    wml[0][wave] = M;
    wml[1][wave] = L;
  }
  __syncthreads();
  const float Mx = fmaxf(fmaxf(wml[0][0], wml[0][1]), fmaxf(wml[0][2], wml[0][3]));
  float sc[4], Lt = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    sc[w] = wml[0][w] == -INFINITY ? 0.f : exp2f(wml[0][w] - Mx);
    Lt += sc[w] * wml[1][w];
  }
  const float inv = Lt != 0.f ? 1.f / Lt : 0.f;
  for (int d = tid; d < D; d += 256)
    Elem<T>::store(out + (int64_t)row * D + d,
                   (sc[0] * red[0][d] + sc[1] * red[1][d] + sc[2] * red[2][d] +
                    sc[3] * red[3][d]) * inv);
}

int num_partitions(int max_ctx, int part_len) {
  return max_ctx <= 0 ? 1 : (max_ctx + part_len - 1) / part_len;
}

// Partition length for the MFMA kernel.  Measured on MI355X: contexts of a
// few thousand tokens stream fastest with long partitions, about one
// wavefront per SIMD (fewer partial results, no reduce-bound tail); long
// and ragged contexts with 512-token partitions (several wavefronts per
// SIMD balance the uneven lengths); small batches need short partitions to
// fill the GPU at all.
// Small batches of short contexts (fewer than 512 items at 256 tokens, at
// most 1024 tokens) take 128-token partitions, up to 8 per (kv head,
// sequence), which one workgroup merges in LDS.
int choose_partition(int num_seqs, int num_kv_heads, int max_ctx, int head_dim, int elem_bytes) {
  const long long units = (long long)num_seqs * num_kv_heads;
  auto items = [&](int p) { return units * ((max_ctx + p - 1) / p); };
  // bf16, 1024 tokens: the config-2 shape then has 2048 wavefronts (four
  // partitions merged per workgroup); measured 159.6-159.9 us against
  // 160.4-160.8 at 2048 tokens.  FP8 (four wavefronts per SIMD, one step in
  // flight each), 512 tokens: 4096 wavefronts, every one resident at once;
  // past 4096 tokens 1024, so that one workgroup still merges a sequence's
  // partitions (eight at most) and no reduce launch is needed.
  const int long_part = elem_bytes == 1 && max_ctx <= 4096 ? 512 : 1024;
  if (max_ctx <= 8192 && items(long_part) >= 1024) return long_part;
  if (items(512) >= 1024) return 512;
  if (items(kPart) < 512 && max_ctx <= 1024 && head_dim <= 128) return kPart / 2;
  return kPart;
}

}  // namespace
}  // namespace pa

using namespace pa;

extern "C" size_t pa_decode_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                           int32_t max_context_len) {
  // Sized for the shortest partition any launch that needs a workspace uses
  // (128 tokens, the f32 group kernel's for small launches), plus two: a
  // balanced launch (contexts above 512 tokens) writes up to
  // ceil(max_context_len / 256) + 3 partial results per row, which that
  // covers; and the shared-prefix group record (6 B + 2 ints).
  const int np = num_partitions(max_context_len, kPart / 2);
  if (np <= 1 || num_seqs <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return (size_t)num_seqs * num_heads * (np + 2) * (head_dim + 2) * sizeof(float) +
         (6 * (size_t)num_seqs + 2) * sizeof(int32_t);
}

namespace {
// The launch configuration pa_decode picks for a call: kernel family,
// partition length and count, and how many partitions one workgroup merges.
struct DecodePlan {
  bool mfma, f32_group;
  bool balanced;  // bf16 launches that would need the reduce: decode_balanced_kernel
  int share_sp;   // balanced: sequences per shared-prefix group (1: no sharing)
  int part_len, np, merge_waves;  // np: partitions, or partial-result slots per row
  size_t ws_bytes;  // workspace the launch needs (0: none)
};
DecodePlan decode_plan(int32_t dtype, bool quantized, int32_t num_seqs, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, int32_t max_context_len) {
  DecodePlan p{};
  const int G = num_heads / num_kv_heads;
  const bool fp8 = dtype == PA_DTYPE_FP8_E4M3;
  p.mfma = !quantized && (dtype == PA_DTYPE_BF16 || fp8) && G <= 16 &&
           (head_dim == 64 || head_dim == 128 || head_dim == 256);
  // f32: the group kernel for head dims that divide 256 (in 4-float steps)
  // and groups of at most kF32MaxG heads, the generic kernel otherwise
  p.f32_group = dtype == PA_DTYPE_F32 && G <= kF32MaxG && head_dim <= 256 &&
                256 % head_dim == 0 && head_dim % 16 == 0;
  p.part_len = p.mfma ? choose_partition(num_seqs, num_kv_heads, max_context_len, head_dim,
                                         fp8 ? 1 : 2)
                      : kPart;
  // f32 group kernel: 128-token partitions when 256-token ones give fewer
  // workgroups than the GPU has CUs
  if (p.f32_group && G <= 8 &&
      (long long)num_seqs * num_kv_heads * num_partitions(max_context_len, kPart) < 256)
    p.part_len = kPart / 2;
  p.np = num_partitions(max_context_len, p.part_len);
  // MFMA kernels: up to 4 partitions (8 for head_dim <= 128) are taken by one
  // workgroup (one wavefront each) and merged in LDS, with no workspace and no
  // reduce launch.
  p.merge_waves = !p.mfma || p.np <= 1 ? 1
                  : p.np == 2           ? 2
                  : p.np <= 4           ? 4
                  : (p.np <= 8 && head_dim <= 128) ? 8
                                                   : 1;
  // Partitioned launches that need the reduce (long, ragged contexts) cut
  // the work evenly over the GPU instead (bf16 caches).
  p.balanced = p.mfma && !fp8 && p.np > 1 && p.merge_waves == 1;
  // A row's slots: a segment of n units meets at most
  // ceil(n / kBalanceMinUnits) + 1 wavefronts (every wavefront holds at
  // least kBalanceMinUnits units), and a row has two segments (shared
  // prefix, private rest) of n <= max_units units in all, so at most
  // ceil(max_units / kBalanceMinUnits) + 3 slots.  Groups of up to 16 / G
  // sequences that begin with the same block share a common prefix of
  // their block tables (one launch of decode_group_kernel finds the groups
  // and prefixes; its record follows the partial results in the
  // workspace).
  p.share_sp = 1;
  if (p.balanced) {
    const int max_units = (max_context_len + 2 * kBlock - 1) / (2 * kBlock);
    p.np = (max_units + kBalanceMinUnits - 1) / kBalanceMinUnits + 3;
    if (G <= 8 && num_seqs >= 2 && num_seqs <= kGroupMaxSeqs) p.share_sp = 16 / G;
  }
  p.ws_bytes = p.np > 1 && p.merge_waves == 1
                   ? (size_t)num_seqs * num_heads * p.np * (head_dim + 2) * sizeof(float) +
                         (p.share_sp > 1 ? (6 * (size_t)num_seqs + 2) * sizeof(int32_t) : 0)
                   : 0;
  return p;
}

int32_t decode_impl(void* out, const void* q, const void* k_cache, const void* v_cache,
                    const float* kv_scales, const int32_t* block_tables,
                    int32_t max_blocks_per_seq, const int32_t* context_lens,
                    int32_t max_context_len, int32_t num_seqs, int32_t num_heads,
                    int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks, float scale,
                    void* workspace, size_t workspace_bytes, int32_t dtype, pa_stream_t stream, int64_t q_row = 0,
                    const uint8_t* block_flags = nullptr) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype) || dtype == PA_DTYPE_FP8_E4M3, PA_ERR_INVALID_ARG,
             "pa_decode: unknown dtype %d", dtype);
  PA_REQUIRE(num_seqs >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 &&
                 num_blocks > 0 && max_blocks_per_seq > 0 && max_context_len >= 0,
             PA_ERR_INVALID_ARG, "pa_decode: bad sizes");
  PA_REQUIRE(num_heads % num_kv_heads == 0, PA_ERR_INVALID_ARG,
             "pa_decode: num_heads %d not a multiple of num_kv_heads %d", num_heads, num_kv_heads);
  PA_REQUIRE((int64_t)max_blocks_per_seq * kBlock >= max_context_len, PA_ERR_OUT_OF_BOUNDS,
             "pa_decode: max_context_len %d exceeds the block table (%d blocks)", max_context_len,
             max_blocks_per_seq);
  PA_REQUIRE(head_dim <= 512, PA_ERR_UNSUPPORTED, "pa_decode: head_dim %d > 512", head_dim);
  if (num_seqs == 0 || max_context_len == 0) return PA_OK;
  PA_REQUIRE(out && q && k_cache && v_cache && block_tables && context_lens, PA_ERR_INVALID_ARG,
             "pa_decode: null pointer");
  const DecodePlan plan = decode_plan(dtype, kv_scales != nullptr, num_seqs, num_heads,
                                      num_kv_heads, head_dim, max_context_len);
  const int G = num_heads / num_kv_heads;
  const bool fp8 = dtype == PA_DTYPE_FP8_E4M3;
  const bool mfma = plan.mfma, f32_group = plan.f32_group;
  const int part_len = plan.part_len, np = plan.np, merge_waves = plan.merge_waves;
  PA_REQUIRE(np <= 1024, PA_ERR_UNSUPPORTED,
             "pa_decode: context of %d tokens needs %d > 1024 partitions", max_context_len, np);
  float* ws_o = nullptr;
  float* ws_ml = nullptr;
  if (plan.ws_bytes) {
    const size_t need = plan.ws_bytes;
    PA_REQUIRE(workspace && workspace_bytes >= need, PA_ERR_WORKSPACE,
               "pa_decode: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    ws_o = (float*)workspace;
    ws_ml = ws_o + (size_t)num_seqs * num_heads * np * head_dim;
  }
  if (q_row == 0) q_row = (int64_t)num_heads * head_dim;
  PA_REQUIRE(q_row >= (int64_t)num_heads * head_dim, PA_ERR_INVALID_ARG,
             "pa_decode: q row stride %lld below num_heads * head_dim", (long long)q_row);
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  const int sp = plan.share_sp;
  int32_t* grp = nullptr;
  if (plan.balanced) {
    if (sp > 1) {
      grp = (int32_t*)(ws_ml + (size_t)num_seqs * num_heads * np * 2);
      decode_group_kernel<<<num_seqs, kGroupThreads, 0, s>>>(
          block_tables, max_blocks_per_seq, context_lens, num_seqs, sp, max_context_len, grp);
    }
#define PA_LAUNCH_BALANCED(DD)                                                                \
  decode_balanced_kernel<DD><<<kBalanceWaves, 64, 0, s>>>(                                    \
      (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, block_tables,   \
      max_blocks_per_seq, context_lens, num_seqs, num_heads, num_kv_heads, G, num_blocks,     \
      scale_log2, np, ws_o, ws_ml, q_row, grp, max_context_len)
    if (head_dim == 64)
      PA_LAUNCH_BALANCED(64);
    else if (head_dim == 128)
      PA_LAUNCH_BALANCED(128);
    else
      PA_LAUNCH_BALANCED(256);
#undef PA_LAUNCH_BALANCED
  } else if (mfma) {
    const dim3 grid(merge_waves > 1 ? 1 : np, num_kv_heads, num_seqs);
    auto* o = (uint16_t*)out;
    auto* qq = (const uint16_t*)q;
#define PA_LAUNCH_MFMA_NW(KERNEL, TC, DD, NW, ...)                                            \
  KERNEL<DD, NW __VA_ARGS__><<<grid, 64 * NW, 0, s>>>(                                                    \
      o, qq, (const TC*)k_cache, (const TC*)v_cache, block_tables, max_blocks_per_seq,        \
      context_lens, num_heads, num_kv_heads, G, num_blocks, scale_log2, np, part_len, ws_o,   \
      ws_ml, q_row, block_flags)
#define PA_LAUNCH_MFMA(KERNEL, TC, DD, ...)                                                   \
  do {                                                                                        \
    if (merge_waves == 2)                                                                     \
      PA_LAUNCH_MFMA_NW(KERNEL, TC, DD, 2, __VA_ARGS__);                                      \
    else if (merge_waves == 4)                                                                \
      PA_LAUNCH_MFMA_NW(KERNEL, TC, DD, 4, __VA_ARGS__);                                      \
    else if (merge_waves == 8)                                                                \
      PA_LAUNCH_MFMA_NW(KERNEL, TC, DD, (DD <= 128 ? 8 : 4), __VA_ARGS__);                    \
    else                                                                                      \
      PA_LAUNCH_MFMA_NW(KERNEL, TC, DD, 1, __VA_ARGS__);                                      \
  } while (0)
    if (fp8 && block_flags) {
      if (head_dim == 64)
        PA_LAUNCH_MFMA(decode_fp8_kernel, uint8_t, 64, , true);
      else if (head_dim == 128)
        PA_LAUNCH_MFMA(decode_fp8_kernel, uint8_t, 128, , true);
      else
        PA_LAUNCH_MFMA(decode_fp8_kernel, uint8_t, 256, , true);
    } else if (fp8) {
      if (head_dim == 64)
        PA_LAUNCH_MFMA(decode_fp8_kernel, uint8_t, 64, , false);
      else if (head_dim == 128)
        PA_LAUNCH_MFMA(decode_fp8_kernel, uint8_t, 128, , false);
      else
        PA_LAUNCH_MFMA(decode_fp8_kernel, uint8_t, 256, , false);
    } else {
      if (head_dim == 64)
        PA_LAUNCH_MFMA(decode_mfma_kernel, uint16_t, 64, );
      else if (head_dim == 128)
        PA_LAUNCH_MFMA(decode_mfma_kernel, uint16_t, 128, );
      else
        PA_LAUNCH_MFMA(decode_mfma_kernel, uint16_t, 256, );
    }
#undef PA_LAUNCH_MFMA
#undef PA_LAUNCH_MFMA_NW
  } else {
    const dim3 grid(np, num_heads, num_seqs);
    if (fp8)
      decode_generic_kernel<uint16_t, Fp8><<<grid, 256, 0, s>>>(
          (uint16_t*)out, (const uint16_t*)q, (const Fp8*)k_cache, (const Fp8*)v_cache,
          block_tables, max_blocks_per_seq, context_lens, num_heads, num_kv_heads, head_dim,
          num_blocks, scale_log2, np, ws_o, ws_ml, nullptr, q_row);
    else if (dtype == PA_DTYPE_BF16)
      decode_generic_kernel<uint16_t><<<grid, 256, 0, s>>>(
          (uint16_t*)out, (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache,
          block_tables, max_blocks_per_seq, context_lens, num_heads, num_kv_heads, head_dim,
          num_blocks, scale_log2, np, ws_o, ws_ml, nullptr, q_row);
    else if (f32_group) {
#define PA_LAUNCH_F32_PL(DD, PL)                                                              \
  decode_f32_group_kernel<DD, PL><<<dim3(np, num_kv_heads, num_seqs), 4 * PL, 0, s>>>(        \
      (float*)out, (const float*)q, (const float*)k_cache, (const float*)v_cache, block_tables, \
      max_blocks_per_seq, context_lens, num_heads, num_kv_heads, num_blocks, scale_log2, np,  \
      ws_o, ws_ml, kv_scales, q_row)
#define PA_LAUNCH_F32(DD)                                                                     \
  (part_len == kPart ? PA_LAUNCH_F32_PL(DD, kPart) : PA_LAUNCH_F32_PL(DD, kPart / 2))
      switch (head_dim) {
        case 16: PA_LAUNCH_F32(16); break;
        case 32: PA_LAUNCH_F32(32); break;
        case 64: PA_LAUNCH_F32(64); break;
        case 128: PA_LAUNCH_F32(128); break;
        default: PA_LAUNCH_F32(256); break;
      }
#undef PA_LAUNCH_F32
#undef PA_LAUNCH_F32_PL
    }
    else
      decode_generic_kernel<float><<<grid, 256, 0, s>>>(
          (float*)out, (const float*)q, (const float*)k_cache, (const float*)v_cache,
          block_tables, max_blocks_per_seq, context_lens, num_heads, num_kv_heads, head_dim,
          num_blocks, scale_log2, np, ws_o, ws_ml, kv_scales, q_row);
  }
  int32_t rc = check_launch("pa_decode");
  if (rc != PA_OK || np == 1 || merge_waves > 1) return rc;
  const dim3 rgrid(num_seqs * num_heads);
  const int bal = plan.balanced ? kBalanceWaves : 0;
#define PA_LAUNCH_REDUCE(TT, DL)                                                              \
  decode_reduce_kernel<TT, DL><<<rgrid, 256, 0, s>>>(                                         \
      (TT*)out, ws_o, ws_ml, context_lens, num_heads, head_dim, np, max_blocks_per_seq,       \
      part_len, bal, num_seqs, num_kv_heads, grp, max_context_len)
  const bool wide = head_dim > 128;
  if (dtype == PA_DTYPE_BF16 || fp8) {
    if (wide)
      PA_LAUNCH_REDUCE(uint16_t, 8);
    else
      PA_LAUNCH_REDUCE(uint16_t, 2);
  } else {
    if (wide)
      PA_LAUNCH_REDUCE(float, 8);
    else
      PA_LAUNCH_REDUCE(float, 2);
  }
#undef PA_LAUNCH_REDUCE
  return check_launch("pa_decode reduce");
}
}  // namespace

extern "C" int32_t pa_decode(void* out, const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* block_tables, int32_t max_blocks_per_seq,
                             const int32_t* context_lens, int32_t max_context_len,
                             int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t num_blocks, float scale, void* workspace,
                             size_t workspace_bytes, int32_t dtype, pa_stream_t stream) {
  return decode_impl(out, q, k_cache, v_cache, nullptr, block_tables, max_blocks_per_seq,
                     context_lens, max_context_len, num_seqs, num_heads, num_kv_heads, head_dim,
                     num_blocks, scale, workspace, workspace_bytes, dtype, stream);
}

extern "C" int32_t pa_decode_fp8_flagged(void* out, const void* q, const void* k_cache,
                                         const void* v_cache, const int32_t* block_tables,
                                         int32_t max_blocks_per_seq, const int32_t* context_lens,
                                         int32_t max_context_len, int32_t num_seqs,
                                         int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t num_blocks, float scale,
                                         void* workspace, size_t workspace_bytes,
                                         const uint8_t* block_flags, pa_stream_t stream) {
  if (!block_flags) {
    clear_error();
    set_error("pa_decode_fp8_flagged: null block_flags");
    return PA_ERR_INVALID_ARG;
  }
  return decode_impl(out, q, k_cache, v_cache, nullptr, block_tables, max_blocks_per_seq,
                     context_lens, max_context_len, num_seqs, num_heads, num_kv_heads, head_dim,
                     num_blocks, scale, workspace, workspace_bytes, PA_DTYPE_FP8_E4M3, stream, 0,
                     block_flags);
}

extern "C" int32_t pa_decode_quantized(void* out, const void* q, const float* k_cache,
                                       const float* v_cache, const float* block_scales,
                                       const int32_t* block_tables, int32_t max_blocks_per_seq,
                                       const int32_t* context_lens, int32_t max_context_len,
                                       int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t num_blocks, float scale,
                                       void* workspace, size_t workspace_bytes,
                                       pa_stream_t stream) {
  if (!block_scales) {
    clear_error();
    set_error("pa_decode_quantized: null block_scales");
    return PA_ERR_INVALID_ARG;
  }
  return decode_impl(out, q, k_cache, v_cache, block_scales, block_tables, max_blocks_per_seq,
                     context_lens, max_context_len, num_seqs, num_heads, num_kv_heads, head_dim,
                     num_blocks, scale, workspace, workspace_bytes, PA_DTYPE_F32, stream);
}

namespace pa {
int32_t decode_strided(void* out, const void* q, int64_t q_row, const void* k_cache,
                       const void* v_cache, const int32_t* block_tables,
                       int32_t max_blocks_per_seq, const int32_t* context_lens,
                       int32_t max_context_len, int32_t num_seqs, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks, float scale,
                       void* workspace, size_t workspace_bytes, int32_t dtype,
                       pa_stream_t stream) {
  return decode_impl(out, q, k_cache, v_cache, nullptr, block_tables, max_blocks_per_seq,
                     context_lens, max_context_len, num_seqs, num_heads, num_kv_heads, head_dim,
                     num_blocks, scale, workspace, workspace_bytes, dtype, stream, q_row);
}
}  // namespace pa

// ---------------------------------------------------------------------------
// pa_decode without a workspace argument: the split-K partial results go to
// `scratch`, a fixed device array of this library (one copy per GPU, alive
// until the process ends).  For callers that cannot allocate (HIP graph
// capture, serving loops that forbid hipMalloc).  Nothing in it needs to
// start at zero: every partition of every sequence writes its record before
// decode_reduce_kernel reads it.  Calls that overlap on one GPU share the
// array and race.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kDecodeScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (host code must use
// it, never the array's name), looked up once per device.
int32_t scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("pa_decode_noalloc: hipGetDevice failed (%s)", hipGetErrorString(e));
    return PA_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("pa_decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d (%s)", dev,
                hipGetErrorString(e));
      return PA_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PA_OK;
}
}  // namespace

extern "C" size_t pa_decode_noalloc_scratch_bytes(void) { return kDecodeScratchBytes; }

extern "C" int32_t pa_decode_noalloc(void* out, const void* q, const void* k_cache,
                                     const void* v_cache, const int32_t* block_tables,
                                     int32_t max_blocks_per_seq, const int32_t* context_lens,
                                     int32_t max_context_len, int32_t num_seqs,
                                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t num_blocks, float scale, int32_t dtype,
                                     pa_stream_t stream) {
  clear_error();
  if (num_seqs > 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 &&
      num_heads % num_kv_heads == 0 && max_context_len > 0) {
    const DecodePlan plan = decode_plan(dtype, false, num_seqs, num_heads, num_kv_heads,
                                        head_dim, max_context_len);
    PA_REQUIRE(plan.ws_bytes <= kDecodeScratchBytes, PA_ERR_WORKSPACE,
               "pa_decode_noalloc: %d sequences x %d heads at context %d need %zu bytes of "
               "split-K scratch, above the fixed %zu (use pa_decode with a workspace)",
               num_seqs, num_heads, max_context_len, plan.ws_bytes, kDecodeScratchBytes);
  }
  // the array used is the current device's: the stream must run there
  if (stream) {
    int cur = -1;
    hipDevice_t sdev = -1;
    PA_REQUIRE(hipGetDevice(&cur) == hipSuccess &&
                   hipStreamGetDevice((hipStream_t)stream, &sdev) == hipSuccess && sdev == cur,
               PA_ERR_INVALID_ARG,
               "pa_decode_noalloc: the stream belongs to device %d, not the current device %d",
               (int)sdev, cur);
  }
  void* ws = nullptr;
  const int32_t rc = scratch_ptr(&ws);
  if (rc != PA_OK) return rc;
  return decode_impl(out, q, k_cache, v_cache, nullptr, block_tables, max_blocks_per_seq,
                     context_lens, max_context_len, num_seqs, num_heads, num_kv_heads, head_dim,
                     num_blocks, scale, ws, kDecodeScratchBytes, dtype, stream);
}
