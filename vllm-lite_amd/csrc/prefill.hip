// Chunked causal prefill attention over the paged KV cache (pa_prefill).
//
// Query row i of sequence s sits at absolute position past[s] + i and
// attends keys 0 .. past[s] + i, all read through the block table.  One
// kernel covers fresh prefill (past = 0) and continuation (past > 0).
//
//  * prefill_mfma_kernel (bf16, D in {64, 128, 256}): each wavefront owns
//    NT * 16 consecutive query rows of one head and streams the keys two
//    16-token blocks at a time.  Sᵀ = K·Qᵀ and Oᵀ = Vᵀ·Pᵀ run on
//    v_mfma_f32_16x16x32_bf16 with the query rows as the N dimension; the
//    lane that receives score (key, row) from the first product is the lane
//    that feeds it to the second, so P never leaves registers.  Online
//    softmax per query row; the causal mask is only evaluated on steps that
//    straddle the diagonal.  Four wavefronts per workgroup cover adjacent
//    row ranges of the same head so their K/V reads share the L1/L2.
//  * prefill_generic_kernel (f32 or bf16, any D <= 512): one wavefront per
//    (query row, head), reference-grade.
#include <algorithm>
#include <type_traits>

#include "pa_common.hpp"
#include "pa_internal.hpp"

namespace pa {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float shfl_xor_f(float x, int mask) { return __shfl_xor(x, mask, 64); }
// Max of three as one v_max3_f32.  fmaxf on values the compiler cannot prove
// canonical gets a quieting v_max_f32 x, x per operand first; MFMA results
// need none (their NaNs are quiet), and the IEEE-mode instruction returns the
// same value fmaxf does for them.  (Measured on the tiled prefill: the eight
// quieting instructions a step cost 1.1%.)
__device__ inline float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// A sequence's query rows and past length as the kernels use them.  The
// offsets are device data: they are clamped to the rows the call owns
// ([0, total_q)) and to max_q rows per sequence (the grid is sized for
// that), and a past outside [0, 2^30] is clamped into it, so inconsistent
// offsets (a caller error) never move a read or write outside q and out.
struct QRange {
  int begin, len, past;
};
__device__ inline QRange q_range(const int32_t* __restrict__ cu_q,
                                 const int32_t* __restrict__ past_lens, int seq, int total_q,
                                 int max_q) {
  const int b = min(max(cu_q[seq], 0), total_q);
  const int e = min(max(cu_q[seq + 1], b), total_q);
  return {b, min(e - b, max_q), min(max(past_lens[seq], 0), 1 << 30)};
}

constexpr int kWaves = 4;
template <int V>
using IC = std::integral_constant<int, V>;

// Lane layout as in decode_mfma_kernel (lane = 16 j + c):
//   QK:  A = K block (row = key c), B = Qᵀ (col = query row c of tile nt)
//        -> lane holds Sᵀ[key 4j + r][row c]
//   PV:  A = Vᵀ (row = dim 16 dt + c), B = Pᵀ, reduction slots 8j + r and
//        8j + 4 + r = key 4j + r of the step's first / second block
//        -> lane holds Oᵀ[dim 16 dt + 4j + r][row c]
template <int D, int NT>
__global__ __launch_bounds__(64 * kWaves) void prefill_mfma_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ past_lens, int Hq, int Hkv,
    int num_blocks, float scale_log2, int64_t q_row, int total_q, int max_q) {
  constexpr int KS = D / 32;
  constexpr int DT = D / 16;
  constexpr int ROWS = 16 * NT;  // query rows per wavefront
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, j = lane >> 4;
  const int h = blockIdx.y, seq = blockIdx.z;
  const int G = Hq / Hkv, kvh = h / G;
  const QRange qr = q_range(cu_q, past_lens, seq, total_q, max_q);
  const int q_begin = qr.begin;
  const int qlen = qr.len;
  const int row0 = (blockIdx.x * kWaves + wave) * ROWS;
  if (row0 >= qlen) return;
  const int past = qr.past;
  const int row_end = min(qlen, row0 + ROWS);
  const int kv_len = min(past + row_end, mbs * kBlock);  // keys this wavefront needs
  const int nblk = (kv_len + kBlock - 1) / kBlock;

  bf16x8 qv[NT][KS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + 16 * nt + c;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (row < qlen)
        qv[nt][s] = *reinterpret_cast<const bf16x8*>(
            q + (int64_t)(q_begin + row) * q_row + (int64_t)h * D + 32 * s + 8 * j);
      else
        qv[nt][s] = bf16x8{};
    }
  }

  f32x4 o[NT][DT];
  float m[NT], lsum[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m[nt] = kNegBig;
    lsum[nt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[nt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int32_t* btab = block_tables + (int64_t)seq * mbs;
  const int64_t head_stride = (int64_t)kBlock * D;
  const int diag_key = past + row0;  // keys above this need the causal test

  for (int ib = 0; ib < nblk; ib += 2) {
    const int kb = ib * kBlock;
    int32_t b0 = btab[ib];
    const bool has1 = ib + 1 < nblk;
    int32_t b1 = has1 ? btab[ib + 1] : b0;
    const int rem = kv_len - kb;
    int lim0 = rem < kBlock ? rem : kBlock;
    int lim1 = has1 ? (rem - kBlock < kBlock ? rem - kBlock : kBlock) : 0;
    if (b0 < 0 || b0 >= num_blocks) { b0 = 0; lim0 = 0; }
    if (b1 < 0 || b1 >= num_blocks) { b1 = 0; lim1 = 0; }

    const uint16_t* k0 = kc + ((int64_t)b0 * Hkv + kvh) * head_stride + c * D + 8 * j;
    const uint16_t* k1 = kc + ((int64_t)b1 * Hkv + kvh) * head_stride + c * D + 8 * j;
    bf16x8 ka[KS], kb8[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      ka[s] = *reinterpret_cast<const bf16x8*>(k0 + 32 * s);
      kb8[s] = *reinterpret_cast<const bf16x8*>(k1 + 32 * s);
    }
    const uint16_t* v0 = vc + ((int64_t)b0 * Hkv + kvh) * head_stride + c * kBlock + 4 * j;
    const uint16_t* v1 = vc + ((int64_t)b1 * Hkv + kvh) * head_stride + c * kBlock + 4 * j;
    uint64_t va[DT], vb[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      va[dt] = *reinterpret_cast<const uint64_t*>(v0 + dt * 16 * kBlock);
      vb[dt] = *reinterpret_cast<const uint64_t*>(v1 + dt * 16 * kBlock);
    }
    const bool partial = lim0 < kBlock || lim1 < kBlock;
    if (partial) {
      const int n0 = min(max(lim0 - 4 * j, 0), 4), n1 = min(max(lim1 - 4 * j, 0), 4);
      const uint64_t mk0 = n0 >= 4 ? ~0ull : ((1ull << (16 * n0)) - 1);
      const uint64_t mk1 = n1 >= 4 ? ~0ull : ((1ull << (16 * n1)) - 1);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        va[dt] &= mk0;
        vb[dt] &= mk1;
      }
    }
    const bool diag = kb + 2 * kBlock - 1 > diag_key;  // wave-uniform

    bf16x8 pb[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s], qv[nt][s], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb8[s], qv[nt][s], s1, 0, 0, 0);
      }
      float x[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = s0[r] * scale_log2;
        x[4 + r] = s1[r] * scale_log2;
      }
      if (partial || diag) {
        const int row_pos = past + row0 + 16 * nt + c;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int k_a = kb + 4 * j + r, k_b = k_a + kBlock;
          if (4 * j + r >= lim0 || k_a > row_pos) x[r] = -INFINITY;
          if (4 * j + r >= lim1 || k_b > row_pos) x[4 + r] = -INFINITY;
        }
      }
      float bm = x[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) bm = fmaxf(bm, x[i]);
      bm = fmaxf(bm, shfl_xor_f(bm, 16));
      bm = fmaxf(bm, shfl_xor_f(bm, 32));
      if (__builtin_amdgcn_ballot_w64(bm > m[nt] + 8.0f)) {
        const float mn = fmaxf(m[nt], bm);
        const float a = fast_exp2(m[nt] - mn);
        m[nt] = mn;
        lsum[nt] *= a;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[nt][dt] *= a;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = fast_exp2(x[i] - m[nt]);
        lsum[nt] += p;
        pb[nt][i] = (__bf16)p;
      }
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint64_t pair[2] = {va[dt], vb[dt]};
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(pair);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[nt], o[nt][dt], 0, 0, 0);
    }
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float l = lsum[nt];
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    const int row = row0 + 16 * nt + c;
    if (row >= qlen) continue;
    const float inv = l != 0.f ? 1.f / l : 0.f;
    uint16_t* orow = out + ((int64_t)(q_begin + row) * Hq + h) * D + 4 * j;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint16_t w[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = f32_to_bf16_bits(o[nt][dt][r] * inv);
      *reinterpret_cast<uint64_t*>(orow + 16 * dt) = *reinterpret_cast<const uint64_t*>(w);
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-tiled MFMA prefill (bf16, D in {64, 128}).
//
// Workgroup = 16 / NT wavefronts sharing one kv head.  Keys are streamed in tiles
// of 64 (4 cache blocks).  Each tile of K and V is copied HBM -> LDS once per
// workgroup with global_load_lds (no register staging) into one of three
// LDS buffers, two tiles ahead of use, and read by all wavefronts.
// Wavefront w owns 16 * NT query rows (NT MFMA column tiles) of one query
// head; with group size G the workgroup covers min(G, 4) heads of the group
// x (256 / min(G, 4)) query tokens, so every K/V byte brought into LDS feeds
// 256 query rows.  NT = 2 keeps a wavefront within 256 registers, so two
// wavefronts share each SIMD and one's softmax overlaps the other's MFMAs.
//
// Per wavefront the 32-key steps form a software pipeline: the Sᵀ = K·Qᵀ
// products of step n + 1 are issued in the same basic block as the
// exponentials and the Oᵀ += Vᵀ·Pᵀ products of step n, so the matrix core
// works while the VALU computes the softmax.  The row max is kept stale
// until a score exceeds it by 2^8; only then (rarely) is the exact max
// formed across lanes and the accumulator rescaled.  The softmax
// denominators are accumulated by one more MFMA per column tile with an
// all-ones operand, which keeps them off the VALU.
//
// LDS layouts (16-byte units, XOR-swizzled so the operand reads of 16 lanes
// hit distinct banks):
//   K tile [64 keys][D]: key row r, 16-byte chunk ch stored at chunk
//     position ch ^ (r % (D / 8)).
//   V tile [4 blocks][D][16]: the two 16-byte halves of a 32-byte dim row d
//     are swapped when bits 2 and 3 of d differ.
//
// Workgroup -> work mapping is XCD-aware: workgroups are dealt round-robin
// to the 8 XCDs, so consecutive logical work items are remapped to the
// same XCD; a logical chunk holds all query tiles of one kv head for all
// sequences, and the tiles that share K/V then share that XCD's L2.  Within
// a chunk the sequences go from most to least work, and within a sequence
// the later (longer) query tiles go first.
template <int D, int NT, typename TC>
__global__ __launch_bounds__(64 * (16 / NT)) void prefill_tiled_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q, const TC* __restrict__ kc,
    const TC* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ past_lens, int Hq, int Hkv,
    int num_blocks, float scale_log2, int B, int tiles_per_seq, int head_groups, int64_t q_row,
    int total_q, int max_q) {
  constexpr int KS = D / 32;   // QK reduction steps
  constexpr int DT = D / 16;   // PV output tiles
  // Cache elements: bf16 (TC = uint16_t) or FP8-E4M3 (TC = uint8_t), the
  // latter converted to bf16 (exactly) as operand fragments are read.
  constexpr bool FP8 = sizeof(TC) == 1;
  constexpr int ES = sizeof(TC);
  constexpr int CPR = D * ES / 16;  // 16-byte chunks per K row
  constexpr int KT = 64;       // keys per LDS tile
  constexpr int W = 16 / NT;   // wavefronts per workgroup (64 query rows x 4 heads)
  constexpr int NBUF = 3;      // LDS tile buffers
  constexpr int TILE_BYTES = KT * D * ES;  // one K (or V) tile
  constexpr int NCH = TILE_BYTES / 1024;   // 1 KB copy chunks per tile
  constexpr int DMA_PER_WAVE = NCH >= W ? NCH / W : 1;
  constexpr int DMA_WAVES = NCH >= W ? W : NCH;  // wavefronts that copy
  constexpr int RPI = 64 / CPR;              // K rows per 1 KB chunk
  constexpr int CPB = D * kBlock * ES / 1024;  // 1 KB chunks per V block
  // 1 KB chunk i of a K tile and of a V tile lie in the same cache block
  // (i / CPB), and a wavefront's chunks stay within one block
  static_assert(RPI * CPB == kBlock && CPB % DMA_PER_WAVE == 0, "one block per wavefront copy");
  // Compute tiles are bf16 for both cache types: an FP8 tile is copied
  // into the staging area `stage` (its own layout, below) and converted to
  // bf16 once per workgroup at the tile boundary, so the per-step fragment
  // reads and the inner loop are those of the bf16 kernel.
  constexpr int CT_BYTES = KT * D * 2;  // one bf16 K (or V) compute tile
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2][NBUF][CT_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t stage[FP8 ? 2 : 1][2][FP8 ? TILE_BYTES : 16];

  const int lane = threadIdx.x & 63;
  const int wave_s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int c = lane & 15, j = lane >> 4;
  const int G = Hq / Hkv;
  const int HW = G < 4 ? G : 4;        // heads per workgroup
  const int TT = 64 * (4 / HW);        // query tokens per workgroup

  // Work items (logical ids): kv head (group) major, then sequences from the
  // most to the least attention work (work = q_len * (past + q_len / 2),
  // ties by index; past 64 sequences the index order), then query tiles
  // longest first.  The items are cut into 8 contiguous chunks, one per XCD
  // (workgroups are dealt round-robin to the XCDs, so workgroup g runs on XCD
  // g % 8), and the items of one chunk stream the same kv head's K/V through
  // that XCD's L2.  The grid is persistent (about one workgroup per CU): the
  // XCD's workgroups take its chunk in rounds of nslot items, the workgroup
  // in slot s taking item s of even rounds and item nslot - 1 - s of odd
  // rounds (within a sequence the tiles go longest first, so this pairs long
  // and short tiles); the workgroups stay on neighbouring items (the same
  // sequence's K/V) and none waits for a CU behind a long-running one.
  const int total = B * Hkv * head_groups * tiles_per_seq;
  const int per_xcd = (total + 7) / 8;
  const int xcd = (int)(blockIdx.x % 8), nslot = (int)(gridDim.x / 8), slot = (int)(blockIdx.x / 8);
  const int lo = min(total, xcd * per_xcd), hi = min(total, lo + per_xcd);
  __shared__ int seq_of_rank[64];
  if (B <= 64 && (int)threadIdx.x < B) {
    auto work = [&](int b) -> long long {
      const QRange r = q_range(cu_q, past_lens, b, total_q, max_q);
      return (long long)r.len * (2 * (long long)r.past + r.len);
    };
    const int b = threadIdx.x;
    const long long wb = work(b);
    int r = 0;
    for (int o2 = 0; o2 < B; ++o2) {
      const long long wo = work(o2);
      r += (wo > wb) || (wo == wb && o2 < b);
    }
    seq_of_rank[r] = b;
  }
  __syncthreads();
  auto seq_of = [&](int rank) -> int { return B <= 64 ? seq_of_rank[rank] : rank; };

  // One work item: attention for one (kv head group, sequence, query tile).
  auto process = [&](int logical) {
  // every wavefront is done with the previous item's LDS tiles
  __syncthreads();
  const int kvhg = logical / (B * tiles_per_seq);
  const int rem = logical % (B * tiles_per_seq);
  const int tile = tiles_per_seq - 1 - rem % tiles_per_seq;
  const int seq = seq_of(rem / tiles_per_seq);
  const int kvh = kvhg / head_groups, hg = kvhg % head_groups;

  const QRange qr = q_range(cu_q, past_lens, seq, total_q, max_q);
  const int q_begin = qr.begin;
  const int qlen = qr.len;
  const int tok0 = tile * TT;
  if (tok0 >= qlen) return;  // uniform over the workgroup
  const int past = qr.past;
  const int key_end = min(past + min(qlen, tok0 + TT), mbs * kBlock);
  const int n_kt = (key_end + KT - 1) / KT;
  const int nblk = (key_end + kBlock - 1) / kBlock;

  const int hl = wave_s % HW, tsub = wave_s / HW;
  const int head_in_group = hg * 4 + hl;
  const bool wave_active = wave_s < HW * (TT / (16 * NT)) && head_in_group < G;
  const int head = kvh * G + head_in_group;
  const int r0 = tok0 + tsub * 16 * NT;  // first query row of this wavefront
  const bool rows_active = wave_active && r0 < qlen;

  bf16x8 qv[NT][KS];
  f32x4 o[NT][DT];
  f32x4 lacc[NT];  // softmax denominators, accumulated on the matrix core
  float nm[NT];  // minus the rows' running maxima (the Sᵀ accumulators start at it)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = r0 + 16 * nt + c;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (rows_active && row < qlen) {
        const bf16x8 raw = *reinterpret_cast<const bf16x8*>(
            q + (int64_t)(q_begin + row) * q_row + (int64_t)head * D + 32 * s + 8 * j);
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[nt][s][i] = (__bf16)((float)raw[i] * scale_log2);
      } else {
        qv[nt][s] = bf16x8{};
      }
    }
    nm[nt] = 0.f;
    lacc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[nt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Block ids.  Each wavefront's HBM -> LDS copies of a tile all read one
  // cache block (block `wblk` of the tile's 4), so a wavefront needs just
  // that id per tile: lane t of `ids` holds it for tile ids_base + t, loaded
  // for 64 tiles at a time with one vector load (at the item's start, then
  // every 64 tiles), and each tile takes it with a lane read.  (A scalar load
  // per tile, through the same counter as the LDS reads, made the step wait
  // for all its LDS reads at the load.)  The index is clamped to
  // the sequence's last block (keys past key_end are masked and their V
  // zeroed) and an id outside the pool reads block 0.  Whether any id of the
  // item's table lies outside the pool is found once per item (`bad_ids`);
  // only then are a tile's per-block validity bits needed (slow path).
  const int32_t* btab = block_tables + (int64_t)seq * mbs;
  const int64_t head_stride = (int64_t)kBlock * D;
  const int wblk = (wave_s * DMA_PER_WAVE) / CPB;
  int bad = 0;
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    const int32_t id = btab[b];
    bad |= (id < 0 || id >= num_blocks) ? 1 : 0;
  }
  const bool bad_ids = __syncthreads_or(bad) != 0;
  auto load_ids = [&](int base) -> int32_t {
    const int t = base + lane;
    if (t >= n_kt) return 0;
    const int32_t id = btab[min(t * (KT / kBlock) + wblk, max(nblk - 1, 0))];
    return (id >= 0 && id < num_blocks) ? id : 0;
  };
  int ids_base = 0;
  int32_t ids = load_ids(0);
  auto fetch_id = [&](int kt) -> int32_t {
    if (kt - ids_base >= 64) {  // wavefront-uniform
      ids_base = kt & ~63;
      ids = load_ids(ids_base);
    }
    return __builtin_amdgcn_readlane(ids, kt - ids_base);
  };
  auto tile_valid = [&](int kt) -> int {
    if (!bad_ids) return (1 << (KT / kBlock)) - 1;
    int v = 0;
#pragma unroll
    for (int b = 0; b < KT / kBlock; ++b) {
      const int bi = kt * (KT / kBlock) + b;
      const int32_t id = bi < nblk ? btab[bi] : -1;
      v |= (id >= 0 && id < num_blocks) ? (1 << b) : 0;
    }
    return v;
  };
  // K row swizzle: 16-byte chunk ch of tile row r sits at chunk position
  // ch ^ kswz(r).  The rows one QK operand read touches (see qk) differ in
  // bits 0-1 and 3-4, which kswz spreads over distinct chunk positions.
  auto kswz = [](int r) -> int {
    constexpr int CPR2 = D * 2 / 16;  // 16-byte chunks per bf16 K row
    return CPR2 >= 16 ? (r & 3) | (((r >> 3) & 3) << 2) : (r & 3) | (((r >> 3) & 1) << 2);
  };
  // V row swizzle: the two 16-byte halves of dim row d are swapped when
  // bit 2 of d is set.  (Measured read rates of the operand pattern, per CU:
  // ~175 B/clk with this swizzle or none, ~100 B/clk when bit 3 takes part.)
  auto vswz = [](int d) -> int { return (d >> 2) & 1; };
  // FP8 K rows (D bytes) are read in 8-byte units (one MFMA fragment); unit
  // u of row r sits at unit position u ^ fsw(r).  Bit 0 is never flipped,
  // so an aligned 16-byte pair of units stays contiguous (one copy lane),
  // and the 32 lanes served together hit distinct bank pairs.  FP8 V dim
  // rows are 16 bytes and need no swizzle.
  auto fsw = [](int r) -> int {
    return D >= 128 ? (((r >> 1) & 1) << 1) | (((r >> 3) & 3) << 2) : ((r >> 3) & 3) << 1;
  };
  // Per-lane element offsets of this wavefront's HBM -> LDS copies (the
  // same for every tile).
  int koff[DMA_PER_WAVE], voff[DMA_PER_WAVE];
#pragma unroll
  for (int i0 = 0; i0 < DMA_PER_WAVE; ++i0) {
    const int i = wave_s * DMA_PER_WAVE + i0;  // 1 KB chunk of the tile
    const int r = i * RPI + lane / CPR;
    if constexpr (FP8) {
      koff[i0] = (r % kBlock) * D + ((lane % CPR) ^ (fsw(r) >> 1)) * 16;
      voff[i0] = ((i % CPB) * 64 + lane) * kBlock;
    } else {
      koff[i0] = (r % kBlock) * D + ((lane % CPR) ^ kswz(r)) * 8;
      const int d = (i % CPB) * 32 + lane / 2;
      voff[i0] = d * kBlock + ((lane & 1) ^ vswz(d)) * 8;
    }
  }
  // Issues this wavefront's share of the HBM -> LDS copies of a key tile
  // into LDS buffer `buf`; `id` is the cache block those copies read.
  auto issue_tile = [&](int32_t id, int buf) {
    const int64_t boff = ((int64_t)id * Hkv + kvh) * head_stride;
    const TC* kbase = kc + boff;
    const TC* vbase = vc + boff;
    if (NCH < W && wave_s >= DMA_WAVES) return;  // the tile has fewer chunks than wavefronts
#pragma unroll
    for (int i0 = 0; i0 < DMA_PER_WAVE; ++i0) {
      const int i = wave_s * DMA_PER_WAVE + i0;
      __builtin_amdgcn_global_load_lds(
          (const void*)(kbase + koff[i0]),
          (__attribute__((address_space(3))) void*)(FP8 ? &stage[buf & 1][0][i * 1024]
                                                        : &smem[0][buf][i * 1024]),
          16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const void*)(vbase + voff[i0]),
          (__attribute__((address_space(3))) void*)(FP8 ? &stage[buf & 1][1][i * 1024]
                                                        : &smem[1][buf][i * 1024]),
          16, 0, 0);
    }
  };
  // A tile that reaches past the last key, or holds a block id outside the
  // pool, has V entries that are not this sequence's data (any bits, NaN
  // included).  Zero them in LDS once, after the tile has landed, so P·V
  // needs no per-step masking (their P is 0 and 0 * 0 = 0).  Uniform over
  // the workgroup; ends with a barrier when it writes.  Returns whether the
  // tile needs key masking.
  auto zero_stale = [&](int kt, int buf, int valid) -> bool {
    const bool special = kt * KT + KT > key_end || valid != (1 << (KT / kBlock)) - 1;
    if (!special) return false;
    uint16_t* vz = reinterpret_cast<uint16_t*>(&smem[1][buf][0]);
    for (int e = threadIdx.x; e < KT * D; e += blockDim.x) {
      const int key = e / D, d = e % D;
      const int b = key / kBlock, t16 = key % kBlock;
      const bool ok = kt * KT + key < key_end && ((valid >> b) & 1);
      if (!ok) {
        const int half = (t16 / 8) ^ vswz(d);
        vz[(b * D + d) * kBlock + half * 8 + t16 % 8] = 0;
      }
    }
    __syncthreads();
    return true;
  };
  // FP8: converts the tile staged in slot `slot` (copy layout: K row r's
  // 8-byte unit u at unit position u ^ fsw(r), V dim rows of 16 bytes) into
  // bf16 compute buffer `buf` (the bf16 layouts and swizzles above), exactly
  // (every E4M3 value is a bf16 value).  All threads of the workgroup.
  // Tile t is staged in slot t % 2 (issue_tile's `buf` is the slot for FP8)
  // and converted one tile boundary before its first use.
  // A wavefront whose units hold a code the hardware conversion reads
  // differently from the reference (NaN / inf / off-OCP codes; never
  // produced from finite input) converts them with the exact integer
  // decode.  Each thread's units are read first, so their LDS reads are in
  // flight together.
  auto convert_tile = [&](int buf, int slot) {
    if constexpr (FP8) {
      constexpr int UPT = KT * D / 8 / (64 * W);  // 8-byte units per thread, K and V each
      static_assert(UPT * 64 * W == KT * D / 8, "tile units per thread");
      uint2 kw[UPT], vw[UPT];
      uint32_t ex = 0;
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int e = threadIdx.x + i * 64 * W;
        const int r = e / (D / 8), u = e % (D / 8);
        kw[i] = *reinterpret_cast<const uint2*>(&stage[slot][0][r * D + (u ^ fsw(r)) * 8]);
        vw[i] = *reinterpret_cast<const uint2*>(&stage[slot][1][e * 8]);  // V dim rows
      }
#pragma unroll
      for (int i = 0; i < UPT; ++i)
        ex |= fp8_exotic_bits(kw[i].x) | fp8_exotic_bits(kw[i].y) | fp8_exotic_bits(vw[i].x) |
              fp8_exotic_bits(vw[i].y);
      auto store = [&](auto exact_c) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
          const int e = threadIdx.x + i * 64 * W;
          const int r = e / (D / 8), u = e % (D / 8);
          const int bd = e / 2, h = e % 2;  // V: bd = block * D + dim
          const int d = bd % D;
          *reinterpret_cast<bf16x8*>(&smem[0][buf][r * (D * 2) + (u ^ kswz(r)) * 16]) =
              decltype(exact_c)::value ? fp8x8_to_bf16_exact(kw[i].x, kw[i].y)
                                       : fp8x8_to_bf16(kw[i].x, kw[i].y);
          *reinterpret_cast<bf16x8*>(&smem[1][buf][bd * 32 + (h ^ vswz(d)) * 16]) =
              decltype(exact_c)::value ? fp8x8_to_bf16_exact(vw[i].x, vw[i].y)
                                       : fp8x8_to_bf16(vw[i].x, vw[i].y);
        }
      };
      if (__builtin_amdgcn_ballot_w64((ex & 0x80808080u) != 0))
        store(std::true_type{});
      else
        store(std::false_type{});
    }
  };
  // Sᵀ for the 32 keys of step ST of the tile in buffer `buf`.  MFMA tile
  // kk's row i holds key 8 (i / 4) + 4 kk + i % 4 of the step, so the lane
  // (c, j) that receives rows 4j .. 4j+3 of both tiles holds keys
  // 8j .. 8j+7: eight consecutive keys of block j / 2.
  auto qk_load = [&](int buf, auto stc, bf16x8 (&ka)[2][KS]) {
    constexpr int ST = decltype(stc)::value;
    const uint8_t* ks = &smem[0][buf][0];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int r = ST * 32 + 8 * (c >> 2) + 4 * kk + (c & 3);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int ch = (4 * s + j) ^ kswz(r);
        ka[kk][s] = *reinterpret_cast<const bf16x8*>(ks + r * (D * 2) + ch * 16);
      }
    }
  };
  auto qk_mfma = [&](const bf16x8 (&ka)[2][KS], f32x4 (&S)[NT][2]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      S[nt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      S[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        S[nt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[0][s], qv[nt][s], S[nt][0], 0, 0, 0);
        S[nt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[1][s], qv[nt][s], S[nt][1], 0, 0, 0);
      }
    }
  };

  bool tile_special;        // current tile needs key masking
  int valid_cur;            // validity bits of the current tile's 4 blocks
  int32_t id_ahead = 0;     // this wavefront's block id of the tile two (FP8: three) ahead
  // Prologue: tiles 0 and 1 in flight, wait for tile 0.  (FP8: tiles 0 and
  // 1 staged and converted, then tile 2 copied into slot 0.)
  issue_tile(fetch_id(0), 0);
  if constexpr (FP8) {
    if (n_kt > 1) issue_tile(fetch_id(1), 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    convert_tile(0, 0);
    if (n_kt > 1) convert_tile(1, 1);
    __syncthreads();
    if (n_kt > 2) issue_tile(fetch_id(2), 0);
  } else if (n_kt > 1) {
    issue_tile(fetch_id(1), 1);
    __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * DMA_PER_WAVE) & 0xF) | (((2 * DMA_PER_WAVE) >> 4) << 14));
  } else {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  }
  __syncthreads();
  valid_cur = tile_valid(0);
  tile_special = zero_stale(0, 0, valid_cur);

  bf16x8 ones;  // all-ones MFMA operand for the row sums
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = (__bf16)1.0f;
  f32x4 S0[NT][2], S1[NT][2];
  {
    bf16x8 ka[2][KS];
    qk_load(0, IC<0>{}, ka);
    qk_mfma(ka, S0);
  }

  // One 32-key step (step ST of tile kt, held in LDS buffer `buf`):
  // softmax of S (already computed), then in one basic block the P·V
  // products of this step and the Sᵀ products of the next.
  auto step = [&](int buf, auto stc, int kt, f32x4 (&S)[NT][2], f32x4 (&Snext)[NT][2]) {
    constexpr int ST = decltype(stc)::value;
    const int next = buf == NBUF - 1 ? 0 : buf + 1;
    const int ahead = next == NBUF - 1 ? 0 : next + 1;
    // This step's Vᵀ fragments (dims 16 dt + c, keys 8j .. 8j+7 = one
    // 16-byte half of the 32-byte row of block 2 ST + j / 2), read first so
    // the softmax covers their latency.
    bf16x8 va[DT];
    {
      const uint8_t* vrow = &smem[1][buf][0] + (2 * ST + (j >> 1)) * (D * 32) + c * 32;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 16 * dt + c;
        va[dt] = *reinterpret_cast<const bf16x8*>(vrow + dt * 16 * 32 + (((j & 1) ^ vswz(d)) * 16));
      }
    }
    // K fragments of the next step, read now so the softmax prep below
    // covers their LDS latency.
    bf16x8 ka[2][KS];
    if constexpr (ST == 0) {
      qk_load(buf, IC<1>{}, ka);
      // this wavefront's block of the tile two ahead, a step before its copy
      if (kt + (FP8 ? 3 : 2) < n_kt) id_ahead = fetch_id(kt + (FP8 ? 3 : 2));
    } else {
      // Tile boundary, at the start of a tile's second step: the next tile
      // has landed (all waves), the buffer two tiles ahead is free again
      // (every wavefront has finished the tile before this one), and the
      // next tile's first K fragments are read now so this step's softmax
      // covers them.  Past the last tile they are read from a buffer of
      // stale data and the products are never used.
      if (kt + 1 < n_kt) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): only tile kt + 1 is in flight
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if constexpr (FP8) {
          // FP8: tile kt + 2 (staged since the last boundary) into the free
          // compute buffer, visible to all at the next boundary's barrier;
          // its staging slot's previous tile (kt + 1) was converted a tile
          // ago, so tile kt + 3 is copied into it
          if (kt + 2 < n_kt) convert_tile(ahead, (kt + 2) & 1);
          if (kt + 3 < n_kt) issue_tile(id_ahead, (kt + 3) & 1);
        } else {
          if (kt + 2 < n_kt) issue_tile(id_ahead, ahead);
        }
      }
      qk_load(next, IC<0>{}, ka);
    }
    {
      const int kb = (2 * kt + ST) * 32;  // first key of this step; x[i] <-> key kb + 8j + i
      if (tile_special || kb + 31 > past + r0) {
        // keys past the end, in invalid blocks, or above a row's diagonal
        const int blk_lim = ((valid_cur >> (2 * ST + (j >> 1))) & 1) ? key_end : 0;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int row_pos = past + r0 + 16 * nt + c;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int key = kb + 8 * j + i;
            if (key >= blk_lim || key > row_pos) S[nt][i >> 2][i & 3] = -INFINITY;
          }
        }
      }
      // S holds log2-domain scores already offset by the row's running
      // max m (the Sᵀ accumulators start at -m).
      float lm[NT];
      bool need = false;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float t0 = max3_raw(S[nt][0][0], S[nt][0][1], S[nt][0][2]);
        const float t1 = max3_raw(S[nt][0][3], S[nt][1][0], S[nt][1][1]);
        lm[nt] = max3_raw(t0, t1, max3_raw(S[nt][1][2], S[nt][1][3], S[nt][1][3]));
        need |= lm[nt] > 8.0f;
      }
      // Rows keep a stale max until one of their scores exceeds it by 2^8;
      // only then is the exact max formed across the four lanes of the row
      // and the accumulator rescaled.  The first step always sets the max
      // (m starts at 0, which says nothing about the row's scores).
      const bool first = ST == 0 && kt == 0;
      if (first || __builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float bm = lm[nt];
          bm = fmaxf(bm, shfl_xor_f(bm, 16));
          bm = fmaxf(bm, shfl_xor_f(bm, 32));
          // a row with every key of the first step masked keeps m = 0
          const float delta = first ? (bm > -INFINITY ? bm : 0.f) : fmaxf(bm, 0.f);
          nm[nt] -= delta;
#pragma unroll
          for (int i = 0; i < 8; ++i) S[nt][i >> 2][i & 3] -= delta;
          if (!first) {
            const float a = fast_exp2(-delta);
            lacc[nt] *= a;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[nt][dt] *= a;
          }
        }
      }
    }

    {
      // The next step's Sᵀ is computed even past this wavefront's last
      // step (it is then unused): keeping it unconditional keeps this one
      // basic block.  Its MFMAs are interleaved by hand with this step's
      // exponentials, one MFMA then EPM exponentials, so the matrix core
      // and the VALU of this wavefront work at the same time.  Consecutive
      // MFMAs go to independent accumulators (s outer, (nt, kk) inner).
      constexpr int NQK = 2 * KS * NT;  // next-step Sᵀ MFMAs
      constexpr int NEXP = 8 * NT;      // exponentials per lane
      constexpr int EPM = NEXP / NQK > 0 ? NEXP / NQK : 1;
      float pv[NT][8];
#pragma unroll
      for (int g = 0; g < NQK; ++g) {
        const int s_ = g / (2 * NT), q_ = g % (2 * NT), nt_ = q_ / 2, kk = q_ % 2;
        Snext[nt_][kk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            ka[kk][s_], qv[nt_][s_], s_ == 0 ? f32x4{nm[nt_], nm[nt_], nm[nt_], nm[nt_]}
                                             : Snext[nt_][kk],
            0, 0, 0);
#pragma unroll
        for (int e = 0; e < EPM; ++e) {
          const int x = g * EPM + e;
          if (x < NEXP) {
            const int nt = x / 8, i = x % 8;
            pv[nt][i] = fast_exp2(S[nt][i >> 2][i & 3]);
          }
        }
      }
#pragma unroll
      for (int x = NQK * EPM; x < NEXP; ++x) {
        const int nt = x / 8, i = x % 8;
        pv[nt][i] = fast_exp2(S[nt][i >> 2][i & 3]);
      }
      // The interleave is imposed on the machine scheduler (compiler passes
      // before it may reorder the exponentials freely): groups of one MFMA
      // then EPM transcendental instructions, in this order.
#pragma unroll
      for (int g = 0; g < NQK; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
        __builtin_amdgcn_sched_group_barrier(0x400, EPM, 0);  // transcendental
      }
      bf16x8 pb[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 8; ++i) pb[nt][i] = (__bf16)pv[nt][i];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], pb[nt], o[nt][dt], 0, 0, 0);
      // Row sums of P: an all-ones operand makes every output row the sum
      // over the 32 keys, from the same bf16 P the numerator uses.
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        lacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[nt], lacc[nt], 0, 0, 0);
    }
    if constexpr (ST == 1) {
      if (kt + 1 < n_kt) {
        valid_cur = tile_valid(kt + 1);
        tile_special = zero_stale(kt + 1, next, valid_cur);
      }
    }
  };

  // Tile kt sits in LDS buffer kt % NBUF.  (Unrolling this loop over the
  // buffers, which would make every LDS address an immediate offset, costs
  // register spills.)
  for (int kt = 0, buf = 0; kt < n_kt; ++kt, buf = buf == NBUF - 1 ? 0 : buf + 1) {
    step(buf, IC<0>{}, kt, S0, S1);
    step(buf, IC<1>{}, kt, S1, S0);
  }

  if (!rows_active) return;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float l = lacc[nt][0];
    const int row = r0 + 16 * nt + c;
    if (row >= qlen) continue;
    const float inv = l != 0.f ? 1.f / l : 0.f;
    uint16_t* orow = out + ((int64_t)(q_begin + row) * Hq + head) * D + 4 * j;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint16_t w[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = f32_to_bf16_bits(o[nt][dt][r] * inv);
      *reinterpret_cast<uint64_t*>(orow + 16 * dt) = *reinterpret_cast<const uint64_t*>(w);
    }
  }
  };
  for (int r = 0; lo + r * nslot < hi; ++r) {
    const int item = lo + r * nslot + ((r & 1) ? nslot - 1 - slot : slot);
    if (item < hi) process(item);
  }
}

// Generic: one wavefront per (query row, head); keys in chunks of 64 with
// an online softmax; lane d accumulates output dims d, d + 64, ...
template <typename T, typename TC = T>
__global__ __launch_bounds__(64) void prefill_generic_kernel(
    T* __restrict__ out, const T* __restrict__ q, const TC* __restrict__ kc,
    const TC* __restrict__ vc, const int32_t* __restrict__ block_tables, int mbs,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ past_lens, int Hq, int Hkv,
    int D, int num_blocks, float scale_log2, const float* __restrict__ kv_scales, int64_t q_row,
    int total_q, int max_q) {
  // kv_scales: per-block scales of a quantised (int8-in-f32) cache, or null
  __shared__ float qs[512];
  __shared__ float ps[64];
  __shared__ int32_t bids[64];
  const int row = blockIdx.x, h = blockIdx.y, seq = blockIdx.z, lane = threadIdx.x;
  const QRange qr = q_range(cu_q, past_lens, seq, total_q, max_q);
  const int q_begin = qr.begin;
  if (row >= qr.len) return;
  const int G = Hq / Hkv, kvh = h / G;
  const int pos = qr.past + row;
  const int64_t qoff = (int64_t)(q_begin + row) * q_row + (int64_t)h * D;
  for (int d = lane; d < D; d += 64) qs[d] = Elem<T>::load(q + qoff + d);
  float acc[8];
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  float m = kNegBig, l = 0.f;
  for (int k0 = 0; k0 <= pos; k0 += 64) {
    __syncthreads();
    if (lane < 4) {
      const int bi = k0 / kBlock + lane;
      int32_t b = (bi < mbs) ? block_tables[(int64_t)seq * mbs + bi] : -1;
      bids[lane] = (b >= 0 && b < num_blocks) ? b : -1;
    }
    __syncthreads();
    const int key = k0 + lane;
    float s = -INFINITY;
    const int32_t b = bids[lane / kBlock];
    if (key <= pos && b >= 0) {
      const TC* kr = kc + (((int64_t)b * Hkv + kvh) * kBlock + key % kBlock) * D;
      const float ks = kv_scales ? kv_scales[b] : 1.0f;
      float a = 0.f;
      for (int d = 0; d < D; ++d) a += qs[d] * (Elem<TC>::load(kr + d) * ks);
      s = a * scale_log2;
    }
    float bm = s;
    for (int w = 32; w > 0; w >>= 1) bm = fmaxf(bm, __shfl_xor(bm, w, 64));
    const float mn = fmaxf(m, bm);
    const float alpha = exp2f(m - mn);
    m = mn;
    const float p = exp2f(s - m);
    float ls = p;
    for (int w = 32; w > 0; w >>= 1) ls += __shfl_xor(ls, w, 64);
    l = l * alpha + ls;
    ps[lane] = p;
    __syncthreads();
    const int nk = min(64, pos + 1 - k0);
    for (int i = 0; i * 64 + lane < D; ++i) {
      const int d = i * 64 + lane;
      float a = acc[i] * alpha;
      for (int t = 0; t < nk; ++t) {
        const int32_t bt = bids[t / kBlock];
        if (bt < 0) continue;
        const float vs = kv_scales ? kv_scales[bt] : 1.0f;
        a += ps[t] * (Elem<TC>::load(vc + (((int64_t)bt * Hkv + kvh) * D + d) * kBlock +
                                     (k0 + t) % kBlock) *
                      vs);
      }
      acc[i] = a;
    }
  }
  const float inv = l != 0.f ? 1.f / l : 0.f;
  for (int i = 0; i * 64 + lane < D; ++i)
    Elem<T>::store(out + ((int64_t)(q_begin + row) * Hq + h) * D + i * 64 + lane, acc[i] * inv);
}

}  // namespace
}  // namespace pa

using namespace pa;



namespace {
// Compute units of the current device (cached per device).
int compute_units() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int32_t prefill_impl(void* out, const void* q, const void* k_cache, const void* v_cache,
                     const float* kv_scales, const int32_t* block_tables,
                     int32_t max_blocks_per_seq, const int32_t* cu_q_lens,
                     const int32_t* past_lens, int32_t num_seqs, int32_t total_q,
                     int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t num_blocks, float scale, int32_t dtype,
                     pa_stream_t stream, int64_t q_row = 0) {
  clear_error();
  PA_REQUIRE(dtype_ok(dtype) || dtype == PA_DTYPE_FP8_E4M3, PA_ERR_INVALID_ARG,
             "pa_prefill: unknown dtype %d", dtype);
  PA_REQUIRE(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_heads > 0 &&
                 num_kv_heads > 0 && head_dim > 0 && num_blocks > 0 && max_blocks_per_seq > 0,
             PA_ERR_INVALID_ARG, "pa_prefill: bad sizes");
  PA_REQUIRE(num_heads % num_kv_heads == 0, PA_ERR_INVALID_ARG,
             "pa_prefill: num_heads %d not a multiple of num_kv_heads %d", num_heads,
             num_kv_heads);
  PA_REQUIRE(head_dim <= 512, PA_ERR_UNSUPPORTED, "pa_prefill: head_dim %d > 512", head_dim);
  if (num_seqs == 0 || total_q == 0 || max_q_len == 0) return PA_OK;
  PA_REQUIRE(out && q && k_cache && v_cache && block_tables && cu_q_lens && past_lens,
             PA_ERR_INVALID_ARG, "pa_prefill: null pointer");
  if (q_row == 0) q_row = (int64_t)num_heads * head_dim;
  PA_REQUIRE(q_row >= (int64_t)num_heads * head_dim, PA_ERR_INVALID_ARG,
             "pa_prefill: q row stride %lld below num_heads * head_dim", (long long)q_row);
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  const bool fp8 = dtype == PA_DTYPE_FP8_E4M3;
  const bool tiled = !kv_scales && (dtype == PA_DTYPE_BF16 || fp8) &&
                     (head_dim == 64 || head_dim == 128);
  const bool mfma = !kv_scales && dtype == PA_DTYPE_BF16 && head_dim == 256;
  if (tiled) {
    const int G = num_heads / num_kv_heads;
    const int HW = G < 4 ? G : 4;
    const int TT = 64 * (4 / HW);
    const int tiles_per_seq = (max_q_len + TT - 1) / TT;
    const int head_groups = (G + 3) / 4;
    const long long total = (long long)num_seqs * num_kv_heads * head_groups * tiles_per_seq;
    PA_REQUIRE(total < (1ll << 31) / 8, PA_ERR_UNSUPPORTED, "pa_prefill: launch too large");
    const int per_xcd = (int)((total + 7) / 8);
    // persistent grid: about one workgroup per CU (a multiple of the 8 XCDs)
    const dim3 grid(8 * std::max(1, std::min(per_xcd, compute_units() / 8)));
    auto* o = (uint16_t*)out;
    auto* qq = (const uint16_t*)q;
    constexpr int NT = 2;
#define PA_LAUNCH_TILED(DD, TC)                                                               \
  prefill_tiled_kernel<DD, NT, TC><<<grid, 64 * (16 / NT), 0, s>>>(                           \
      o, qq, (const TC*)k_cache, (const TC*)v_cache, block_tables, max_blocks_per_seq,        \
      cu_q_lens, past_lens, num_heads, num_kv_heads, num_blocks, scale_log2, num_seqs,        \
      tiles_per_seq, head_groups, q_row, total_q, max_q_len)
    if (fp8) {
      if (head_dim == 128)
        PA_LAUNCH_TILED(128, uint8_t);
      else
        PA_LAUNCH_TILED(64, uint8_t);
    } else {
      if (head_dim == 128)
        PA_LAUNCH_TILED(128, uint16_t);
      else
        PA_LAUNCH_TILED(64, uint16_t);
    }
#undef PA_LAUNCH_TILED
  } else if (mfma) {
    constexpr int NT = 2;
    const int rows_per_wg = 16 * NT * kWaves;
    const dim3 grid((max_q_len + rows_per_wg - 1) / rows_per_wg, num_heads, num_seqs);
    auto* o = (uint16_t*)out;
    auto* qq = (const uint16_t*)q;
    auto* kc = (const uint16_t*)k_cache;
    auto* vc = (const uint16_t*)v_cache;
#define PA_LAUNCH_PREFILL(DD)                                                                 \
  prefill_mfma_kernel<DD, NT><<<grid, 64 * kWaves, 0, s>>>(                                   \
      o, qq, kc, vc, block_tables, max_blocks_per_seq, cu_q_lens, past_lens, num_heads,       \
      num_kv_heads, num_blocks, scale_log2, q_row, total_q, max_q_len)
    PA_LAUNCH_PREFILL(256);
#undef PA_LAUNCH_PREFILL
  } else {
    const dim3 grid(max_q_len, num_heads, num_seqs);
    if (dtype == PA_DTYPE_FP8_E4M3)
      prefill_generic_kernel<uint16_t, Fp8><<<grid, 64, 0, s>>>(
          (uint16_t*)out, (const uint16_t*)q, (const Fp8*)k_cache, (const Fp8*)v_cache,
          block_tables, max_blocks_per_seq, cu_q_lens, past_lens, num_heads, num_kv_heads,
          head_dim, num_blocks, scale_log2, nullptr, q_row, total_q, max_q_len);
    else if (dtype == PA_DTYPE_BF16)
      prefill_generic_kernel<uint16_t><<<grid, 64, 0, s>>>(
          (uint16_t*)out, (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache,
          block_tables, max_blocks_per_seq, cu_q_lens, past_lens, num_heads, num_kv_heads,
          head_dim, num_blocks, scale_log2, nullptr, q_row, total_q, max_q_len);
    else
      prefill_generic_kernel<float><<<grid, 64, 0, s>>>(
          (float*)out, (const float*)q, (const float*)k_cache, (const float*)v_cache,
          block_tables, max_blocks_per_seq, cu_q_lens, past_lens, num_heads, num_kv_heads,
          head_dim, num_blocks, scale_log2, kv_scales, q_row, total_q, max_q_len);
  }
  return check_launch("pa_prefill");
}
}  // namespace

extern "C" int32_t pa_prefill(void* out, const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_tables, int32_t max_blocks_per_seq,
                              const int32_t* cu_q_lens, const int32_t* past_lens,
                              int32_t num_seqs, int32_t total_q, int32_t max_q_len,
                              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              int32_t num_blocks, float scale, int32_t dtype, pa_stream_t stream) {
  return prefill_impl(out, q, k_cache, v_cache, nullptr, block_tables, max_blocks_per_seq,
                      cu_q_lens, past_lens, num_seqs, total_q, max_q_len, num_heads, num_kv_heads,
                      head_dim, num_blocks, scale, dtype, stream);
}

extern "C" int32_t pa_prefill_quantized(void* out, const void* q, const float* k_cache,
                                        const float* v_cache, const float* block_scales,
                                        const int32_t* block_tables, int32_t max_blocks_per_seq,
                                        const int32_t* cu_q_lens, const int32_t* past_lens,
                                        int32_t num_seqs, int32_t total_q, int32_t max_q_len,
                                        int32_t num_heads, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t num_blocks, float scale,
                                        pa_stream_t stream) {
  if (!block_scales) {
    clear_error();
    set_error("pa_prefill_quantized: null block_scales");
    return PA_ERR_INVALID_ARG;
  }
  return prefill_impl(out, q, k_cache, v_cache, block_scales, block_tables, max_blocks_per_seq,
                      cu_q_lens, past_lens, num_seqs, total_q, max_q_len, num_heads, num_kv_heads,
                      head_dim, num_blocks, scale, PA_DTYPE_F32, stream);
}

namespace pa {
int32_t prefill_strided(void* out, const void* q, int64_t q_row, const void* k_cache,
                        const void* v_cache, const int32_t* block_tables,
                        int32_t max_blocks_per_seq, const int32_t* cu_q_lens,
                        const int32_t* past_lens, int32_t num_seqs, int32_t total_q,
                        int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t num_blocks, float scale, int32_t dtype,
                        pa_stream_t stream) {
  return prefill_impl(out, q, k_cache, v_cache, nullptr, block_tables, max_blocks_per_seq,
                      cu_q_lens, past_lens, num_seqs, total_q, max_q_len, num_heads, num_kv_heads,
                      head_dim, num_blocks, scale, dtype, stream, q_row);
}
}  // namespace pa
