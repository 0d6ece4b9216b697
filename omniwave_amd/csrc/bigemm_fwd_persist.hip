// Persistent BiGEMM forward for d = 128, rd = 256 with contiguous channel groups (radix level 0,
// or one group) or the strided groups of radix levels >= 1 (q_c in {2, 4, 8}), and 16-byte
// aligned rows: the 14x14x512 and 7x7x1024 stages of OmniWeave-T.
//
// Same math and operand packing as bigemm_fwd.hip (reference omniweave/ops/reference.py:147-171;
// operand scheme in ow_device.h).  Organisation:
//   * one workgroup of eight waves per CU (149 KB of LDS), persistent over units of up to 8
//     32-token pairs (256 token rows, one pair per wave) x one channel group.  With at most one
//     unit per CU each workgroup runs one unit.  With more, contiguous groups take whole units
//     round robin, and every workgroup of an XCD (dispatched round-robin over the 8 XCDs) keeps
//     one channel group, so an XCD's L2 holds one group's weights; strided groups split each
//     group's pairs evenly over grid / q_c workgroups, which run their range as full units and
//     one partial last unit whose waves without a pair compute nothing, so that the last
//     round's 2-byte stores come from every XCD;
//   * the eight waves share one stream of weight chunks (24 KB per 32-row chunk of the expanded
//     dimension, three LDS buffers, copied global -> LDS with global_load_lds), with the chunk
//     loop of bigemm_fwd.hip: chunk ec + 1's U'/V' products issued with chunk ec's gate values
//     between them, then chunk ec's W += Z B_o;
//   * the x tile is copied straight into LDS (buffer_load ... lds; pad tokens read as zero): each
//     wave loads, and later reads, only its own 32 rows, so the tile needs no workgroup
//     barrier.  A wave's rows of the next unit are requested as soon as its output phase has
//     read the current rows for the residual, and land while the stores and the next unit's
//     first chunk copy are in flight;
//   * the RMSNorm row scales come from a statistics buffer (a separate pass) or from the
//     previous block's per-group sums of squares (chained statistics): the tile holds only the
//     unit's own channel group; strided groups read whole rows anyway and form the scales from
//     them when neither is given;
//   * the output: delta = A_o W, rounded (and scaled by the drop-path factor), is staged per
//     wave in the chunk buffers that the loop no longer reads, and stored as 16-byte row pieces
//     with the residual round(x + delta), x from the tile.
// Tile layout: row r holds its 128 channels, 16-byte piece p at slot p ^ tile128_swz(r), so
// the rows of a token-side transposed read hit different LDS banks.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "ow_device.h"

namespace ow {
namespace {

constexpr int kD = 128;
constexpr int kRD = 256;
constexpr int kKS = kD / 16;             // 16-deep K steps over the channel group
constexpr int kMB = kD / 32;             // 32-channel output blocks
constexpr int kNCH = kRD / 32;           // 32-row chunks of the expanded dimension
constexpr int kFrU = kKS;                // B_u'^T fragments per chunk (B_v'^T the same)
constexpr int kFrO = 2 * kMB;            // B_o fragments per chunk
constexpr int kFrCh = 2 * kFrU + kFrO;   // 24 fragments = 24 KB per chunk
constexpr int kChElems = kFrCh * kFragElems;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = 32 * kWaves;       // 256 rows per unit
constexpr int kGroups = kRows / kG;      // 16 token groups per unit
constexpr int kTileOps = 32 * kD * 2 / 1024;  // 1 KB tile copies per wave (8)
constexpr int kLdo = kD + 8;             // output staging row stride (elements)
constexpr int kTokLds = 512;             // token-table entries kept in LDS (q_s <= 32)

struct PersistLds {
  uint16_t x[kRows * kD];              // the unit's tile, 64 KB
  uint16_t w[3][kChElems];             // weight chunk buffers, after the chunk loop the output staging
  int32_t rowid[2][kRows];             // per unit (double-buffered): input row, -1 for pad rows
  int32_t rowout[2][kRows];            // output row, -1: not stored
  float rsc[2][kRows];                 // RMSNorm scale of each row
  float dsc[2][kGroups];               // drop-path scale of each token group
  u32x4 tok_ops[3][64];                // token-side operand rows (A_u, A_v, A_o), read per unit
  int32_t tok[kTokLds];                // the token table when it has at most kTokLds entries
  int32_t out_tok[kTokLds];            // the output-row table (same bound)
};
static_assert(32 * kLdo * 2 * kWaves <= 3 * kChElems * 2, "output staging fits in the chunk buffers");

// Strided channel groups (radix levels >= 1: group qc is channels res + t NS, t < 128, NS = q_c):
// a 16-byte piece of a row holds M = 8 / NS columns of every group, so the tile comes through
// registers.  strided_fetch loads a wave's whole rows, NS pieces per lane and row (16 lanes per
// row, 4 rows per pass, passes p0 .. p0 + NP - 1); strided_write keeps the group's columns
// (strided_pack) at the tile's swizzled positions.
template <int NS, int NP>
__device__ __forceinline__ void strided_fetch(__amdgpu_buffer_rsrc_t rx, const int32_t* rowid, int channels, int lane,
                                              int p0, u32x4 (&v)[NP][NS]) {
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int32_t id = rowid[4 * (p0 + p) + (lane >> 4)];
    const uint32_t off =
        id >= 0 ? static_cast<uint32_t>(id) * static_cast<uint32_t>(channels * 2) + 16u * (lane & 15) : kOffOut;
#pragma unroll
    for (int j = 0; j < NS; ++j) v[p][j] = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 256u * j, 0, 0);
  }
}
template <int NS, int NP>
__device__ __forceinline__ void strided_write(uint16_t* xw, int lane, int res, int p0, const u32x4 (&v)[NP][NS]) {
  constexpr int M = 8 / NS;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int r = 4 * (p0 + p) + (lane >> 4);  // row of the wave
    const int sw = 8 * tile128_swz(r);          // the swizzle in channels
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int c0 = M * ((lane & 15) + 16 * j);
      const StridedPack<M> e = strided_pack<M>(v[p][j], res);
      uint16_t* dst = xw + r * kD + (c0 ^ sw);
      if constexpr (M == 1)
        *dst = static_cast<uint16_t>(e);
      else
        *reinterpret_cast<StridedPack<M>*>(dst) = e;
    }
  }
}

// Token-table entries of one row of a unit (loads only: consumed by meta_write a phase later).
struct TokLoad {
  int32_t t, to, b;
  float ds;
};

// F8: V' = P_v B_v'' on the K = 64 e4m3 MFMA (ow_device.h, fp8 channel side); a chunk is then
// f8_chunk_units(128) = 20 copy units, which waves 0-3 copy three of and waves 4-7 two of.
// NS: 1 for contiguous channel groups (tile rows by DMA), else the channel stride of the
// strided groups (q_c = NS; whole rows through registers, QW = NS pieces per lane and row, which
// also give the RMSNorm scales; output by 2-byte stores).
// Scheduling (a unit is up to 8 consecutive 32-token pairs of one channel group, pair p = token
// groups 2p, 2p + 1): n_pairs == 0: one unit per workgroup, unit u = pairs 8 (u / q_c) .. + 7
// of group u % q_c (the grid covers the n_units units); n_pairs < 0: the grid is a multiple of
// 8 and of q_c, and workgroup b runs units b, b + grid, ... (contiguous groups); n_pairs > 0: the
// same grid, and each channel group's n_pairs pairs are split evenly over its grid / q_c
// workgroups, which run their range as full units and one partial last unit (strided groups).
template <class Ty, bool F8, int NS>
__global__ void __launch_bounds__(kThreads) bigemm_fwd_persist_kernel(PersistArgs a, int32_t n_units, int32_t n_pairs) {
  constexpr int QW = NS > 1 ? NS : 0;  // register-tile fetch width (0: DMA tile)
  constexpr int SNP = QW == 8 ? 1 : 2;  // register tiles: passes (4 rows each) per batch
  constexpr int CHU = F8 ? f8_chunk_units(kD) : kFrCh;      // 1 KB copy units per chunk
  constexpr int CH_ELEMS = CHU * kFragElems;
  constexpr int HEAD = F8 ? kF8HeadBytes / 2 : kHeadElems;  // packed head, 16-bit elements
  constexpr int F8_BV = kFrU;                                // fp8: first unit of B_v'^T (K = 64)
  constexpr int F8_BO = kFrU + 2 * (kD / 64);                // fp8: first unit of B_o
  static_assert(CHU <= kFrCh && CHU > 2 * kWaves, "two or three copy units per wave");
  __shared__ __attribute__((aligned(16))) PersistLds sh;
  // lane and wave are re-read opaquely at the top of every unit (see the loop): the compiler
  // would otherwise compute hundreds of per-lane addresses once, before the loop, and keep them
  // live (spilled) through it.
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int hh = lane >> 5, l32 = lane & 31;
  uint32_t lane16 = 16u * static_cast<uint32_t>(lane);
  const uint32_t xbytes = static_cast<uint32_t>(static_cast<int64_t>(a.batch) * a.n_tok * a.channels * 2);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, xbytes);
  const int64_t n_groups = static_cast<int64_t>(a.batch) * a.q_s;
  const bool tok_lds = a.q_s * kG <= kTokLds;  // token tables copied to LDS at the start

  // This workgroup's channel group qc and 32-token pairs [p_lo, p_hi).  Contiguous groups: all
  // workgroups of an XCD (dispatched round-robin over the 8 XCDs) are of one group, so an XCD's
  // L2 holds one group's weights.  Strided groups: the q_c workgroups of one pair range run on
  // one XCD, so their whole-row reads and the 2-byte stores of their interleaved columns meet in
  // one L2.
  int qc;
  int32_t p_lo, p_hi;
  int32_t p_step = kWaves;  // pairs from one of the workgroup's units to the next
  if (n_pairs <= 0) {
    int32_t u = blockIdx.x;
    if constexpr (QW > 0) {
      const int nwg = gridDim.x, xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
      const int per = nwg >> 3, rem = nwg & 7;
      u = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + slot;
    }
    if (u >= n_units) return;
    qc = u % a.q_c;
    p_lo = (u / a.q_c) * kWaves;
    p_hi = p_lo + kWaves;
    if (n_pairs < 0) {  // units u + j grid: the same group, pairs 8 grid / q_c further each
      p_step = kWaves * static_cast<int32_t>(gridDim.x / a.q_c);
      p_hi = (n_units / a.q_c) * kWaves;
    }
  } else {
    const int nwg = gridDim.x, per = nwg >> 3, xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    int k;
    if (QW > 0 || 8 % a.q_c != 0) {
      const int idx = QW > 0 ? xcd * per + slot : static_cast<int>(blockIdx.x);
      qc = idx % a.q_c;
      k = idx / a.q_c;
    } else {  // contiguous groups, q_c dividing 8: one group per XCD
      qc = xcd % a.q_c;
      k = (xcd / a.q_c) * per + slot;
    }
    const int64_t wg = nwg / a.q_c;
    p_lo = static_cast<int32_t>(k * static_cast<int64_t>(n_pairs) / wg);
    p_hi = static_cast<int32_t>((k + 1) * static_cast<int64_t>(n_pairs) / wg);
    if (p_lo >= p_hi) return;
  }
  // The group's first channel mod NS (its residue; strided groups).
  const int res_g = NS > 1 ? (a.chan[qc * kD] & (NS - 1)) : 0;

  // Row l < 32 of this wave in the unit of pairs p0 .. p0 + np - 1 (lanes < 32): the token-table
  // loads of meta_write.  Waves past the unit's pairs get pad rows.
  auto meta_load = [&](int32_t p0, int np) {
    TokLoad e{-1, -1, -1, 1.0f};
    if (lane < 32 && wave < np) {
      const int64_t tg = 2 * (static_cast<int64_t>(p0) + wave) + (lane >> 4);
      if (tg < n_groups) {
        e.b = static_cast<int32_t>(tg / a.q_s);
        const int32_t sg = static_cast<int32_t>(tg - static_cast<int64_t>(e.b) * a.q_s);
        const int ti = sg * kG + (lane & 15);
        if (tok_lds) {
          e.t = sh.tok[ti];
          if (a.out_tok) e.to = sh.out_tok[ti];
        } else {
          e.t = a.tok[ti];
          if (a.out_tok) e.to = a.out_tok[ti];
        }
        if (a.drop_scale) e.ds = a.drop_scale[e.b];
      }
    }
    return e;
  };
  // Input / output rows and drop-path scales of this wave's rows, slot s; returns the lane's
  // input row (-1: pad token or past the batch).
  auto meta_write = [&](const TokLoad& e, int s) {
    int32_t id = -1, od = -1;
    if (lane < 32) {
      if (e.b >= 0 && e.t >= 0 && e.t < a.n_tok) {
        id = e.b * a.n_tok + e.t;
        od = id;
        if (a.out_tok) od = (e.to >= 0 && e.to < a.n_tok) ? e.b * a.n_tok + e.to : -1;
      }
      sh.rowid[s][32 * wave + lane] = id;
      sh.rowout[s][32 * wave + lane] = od;
      if ((lane & 15) == 0) sh.dsc[s][2 * wave + (lane >> 4)] = e.ds;
    }
    wave_lds_sync();
    return id;
  };
  // kNormBuffer: the row's scale; kNormPartials: the sum of its partial sums of squares.
  auto stats_load = [&](int32_t id) {
    float v = 0.0f;
    if (lane < 32 && id >= 0) {
      if (a.norm == kNormBuffer) {
        v = a.row_scale[id];
      } else if (a.norm == kNormPartials) {
        for (int q = 0; q < a.parts; ++q) v += a.row_scale[static_cast<int64_t>(id) * a.parts + q];
      }
    }
    return v;
  };
  auto stats_write = [&](float v, int32_t id, int s) {
    if (lane < 32 && a.norm != kNormInline) {  // kNormInline: strided_tile writes the scales
      float r = 1.0f;
      if (id >= 0 && a.norm == kNormBuffer) r = v;
      if (id >= 0 && a.norm == kNormPartials) r = rms_scale<Ty>(v / static_cast<float>(a.channels), a.eps);
      sh.rsc[s][32 * wave + lane] = r;
    }
  };
  // This wave's 32 tile rows of slot s: copy k covers rows 4k .. 4k + 3, lane -> row
  // 4k + lane / 16, slot lane % 16, which holds the row's piece (lane % 16) ^ tile128_swz(row).
  auto issue_tile = [&](int s) {
    const uint32_t col0 = static_cast<uint32_t>(qc * kD * 2);
#pragma unroll
    for (int k = 0; k < kTileOps; ++k) {
      const int r = 32 * wave + 4 * k + (lane >> 4);
      const int32_t id = sh.rowid[s][r];
      const uint32_t piece = static_cast<uint32_t>((lane & 15) ^ tile128_swz(r));
      const uint32_t voff = id >= 0 ? static_cast<uint32_t>(id) * static_cast<uint32_t>(a.channels * 2) + col0 + 16u * piece
                                    : kOffOut;
      tile_copy(rx, voff, lds_addr(&sh.x[(32 * wave_u + 4 * k) * kD]));
    }
  };
  auto issue_chunk = [&](int ec) {
    const uint16_t* src = uniform_ptr(a.packed + HEAD + (static_cast<size_t>(qc) * kNCH + ec) * CH_ELEMS);
    uint16_t* dst = sh.w[ec % 3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int f = wave_u + i * kWaves;
      if (f < CHU) copy_frag_to_lds(src + f * kFragElems, dst + f * kFragElems, lane16);
    }
  };
  // Waits until at most this wave's copies of one chunk plus E younger operations are
  // outstanding.
  auto wait_chunk = [&](auto e_tag) {
    constexpr int E = decltype(e_tag)::value;
    if (F8 && wave_u >= CHU - 2 * kWaves)
      wait_vmcnt<2 + E>();
    else
      wait_vmcnt<3 + E>();
  };
  using E0 = std::integral_constant<int, 0>;

  // Register tiles (QW > 0), one batch of passes p0 .. p0 + SNP - 1: tile_fetch issues the loads
  // of whole rows (16 lanes per row), tile_put writes the group's columns to the tile and, with
  // kNormInline, the rows' RMSNorm scales: sum of squares over the 16 lanes (DPP), the total in
  // lane 15 of the row.
  using TileBatch = u32x4[SNP][QW > 0 ? QW : 1];
  auto tile_fetch = [&](int ss, int p0, TileBatch& v) {
    if constexpr (QW > 0) strided_fetch<NS, SNP>(rx, &sh.rowid[ss][32 * wave], a.channels, lane, p0, v);
  };
  auto tile_put = [&](int ss, int p0, const TileBatch& v) {
    if constexpr (QW > 0) {
      strided_write<NS, SNP>(sh.x + 32 * wave * kD, lane, res_g, p0, v);
      if (a.norm == kNormInline) {
#pragma unroll
          for (int p = 0; p < SNP; ++p) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < QW; ++j)
#pragma unroll
              for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(v[p][j][e], acc);
            acc = group_sum<16>(acc);
            if ((lane & 15) == 15) {
              const int r = 32 * wave + 4 * (p0 + p) + (lane >> 4);
              sh.rsc[ss][r] =
                  sh.rowid[ss][r] >= 0 ? rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps) : 1.0f;
            }
          }
      }
    }
  };
  // The whole register tile of unit uu, slot ss (after the unit's stores; batch 0 already
  // requested into va): each batch's loads go out before the previous batch is put (two batches
  // of registers in flight).
  auto strided_tile = [&](int ss, TileBatch& va) {
    if constexpr (QW > 0) {
      TileBatch vb;
#pragma unroll
      for (int p0 = 0; p0 < 8; p0 += 2 * SNP) {
        tile_fetch(ss, p0 + SNP, vb);
        tile_put(ss, p0, va);
        if (p0 + 2 * SNP < 8) tile_fetch(ss, p0 + 2 * SNP, va);
        tile_put(ss, p0 + SNP, vb);
      }
      wave_lds_sync();
    }
  };
  int s = 0;
  int32_t pu = p_lo;  // the unit's first pair
  if (wave < 3) sh.tok_ops[wave][lane] = reinterpret_cast<const u32x4*>(a.packed)[wave * 64 + lane];
  if (tok_lds) {
    for (int i = threadIdx.x; i < a.q_s * kG; i += kThreads) {
      sh.tok[i] = a.tok[i];
      if (a.out_tok) sh.out_tok[i] = a.out_tok[i];
    }
  }
  __syncthreads();
  {
    const int32_t id = meta_write(meta_load(pu, p_hi - pu < kWaves ? p_hi - pu : kWaves), 0);
    if constexpr (QW == 0) issue_tile(0);
    issue_chunk(0);
    TileBatch va0;
    tile_fetch(0, 0, va0);
    strided_tile(0, va0);
    stats_write(stats_load(id), id, 0);
    wave_lds_sync();
    wait_chunk(E0{});  // this wave's tile rows; chunk 0 may still be in flight
  }

#pragma unroll 1
  for (; pu < p_hi; pu += p_step, s ^= 1) {
    asm volatile("" : "+v"(lane), "+v"(wave));
    hh = lane >> 5;
    l32 = lane & 31;
    lane16 = 16u * static_cast<uint32_t>(lane);
    const int np = p_hi - pu < kWaves ? p_hi - pu : kWaves;  // the unit's pairs
    const int32_t pn = pu + p_step;
    const bool has_next = pn < p_hi;
    const int np_next = p_hi - pn < kWaves ? p_hi - pn : kWaves;
    // Strided groups: a wave with no pair in this unit (a partial last unit, or pad token groups
    // only) copies its share of the weight chunks and meets the barriers, but computes nothing;
    // such a unit is the last of the workgroup's range.  (Contiguous groups compute pad rows as
    // zeros instead: the branches cost their chunk loop more than the idle waves give back.)
    const bool act = NS == 1 || (wave_u < np && 2 * (static_cast<int64_t>(pu) + wave_u) < n_groups);
    TokLoad en{-1, -1, -1, 1.0f};
    if (has_next) en = meta_load(pn, np_next);  // consumed after the token side

    // Token side of this wave's pair (rows 32 wave .. + 31 of the tile).
    constexpr int KV = F8 ? kKS / 4 : kKS;
    using VOp = std::conditional_t<F8, u32x8, u32x4>;
    u32x4 Pu[kKS], xk[kKS / 2][2];
    VOp Pv[KV];
    if (act) {
      // The token operands are read per unit from LDS rather than kept live through the loop.
      const u32x4 fAu = sh.tok_ops[0][lane];
      const u32x4 fAv = sh.tok_ops[1][lane];
      // X^T operands by transposed reads; channel c of tile row r sits at c ^ 8 tile128_swz(r).
      const uint32_t xb = lds_addr(sh.x) + 2u * static_cast<uint32_t>(32 * kD * wave);
      pair_xt_tr<kKS>(
          [&](int r, int c) { return xb + 2u * static_cast<uint32_t>(r * kD + (c ^ (8 * tile128_swz(r)))); }, lane,
          xk);
      u32x4 bu = fAu, bv = fAv;
      if (a.norm != kNormNone) {
        const float* r8 = &sh.rsc[s][32 * wave + 16 * ((lane >> 4) & 1) + 4 * hh];
        bu = scale8<Ty>(fAu, r8);
        if constexpr (F8) {  // P_v comes out quantised: the multiplier is in the token operand
          const float qv = reinterpret_cast<const float*>(a.packed + kHeadElems)[kF8QuantPv];
          bv = scale8m<Ty>(fAv, r8, qv);
        } else {
          bv = scale8<Ty>(fAv, r8);
        }
      }
      if constexpr (F8)
        pair_token_side_f8_mma<Ty, kKS>(xk, bu, bv, lane, Pu, Pv);
      else
        pair_token_side_mma<Ty, kKS>(xk, bu, bv, lane, Pu, Pv);
    }
    int32_t id_next = -1;
    if (has_next) id_next = meta_write(en, s ^ 1);

    // Chunk 0 has landed for every wave; chunks 1 and 2 go out, then the next unit's statistics
    // input (consumed at the end of this unit; younger than the copies, so the chunk waits below
    // stay exact).
    wait_lds_dma();
    __syncthreads();
    issue_chunk(1);
    issue_chunk(2);
    float snext = 0.0f;
    if (has_next) snext = stats_load(id_next);

    f32x16 W[kMB];
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) W[mb][i] = 0.0f;

    // Chunk loop (as bigemm_fwd.hip's pipelined loop): one step issues chunk ec + 1's U'/V'
    // products and chunk ec's W += Z B_o, their fragments read DEPTH ahead, with one gate value
    // of chunk ec computed after each U'/V' product.
    constexpr int DEPTH = 4;
    auto stream = [&](auto nu_tag, auto no_tag, uint32_t bn, uint32_t bo, f32x16& Un, f32x16& Vn,
                      const f32x16& Uc, const f32x16& Vc) {
      constexpr int NU = decltype(nu_tag)::value;  // U'/V' fragments of chunk ec + 1 (0 or 2 KS)
      constexpr int NO = decltype(no_tag)::value;  // B_o fragments of chunk ec (0 or kFrO)
      constexpr int NF = NU + NO;
      static_assert(NO == 0 || NU == 0 || NU == 16, "one gate value per U'/V' product");
      auto read = [&](auto ic) -> u32x4 {
        constexpr int i = decltype(ic)::value;
        if constexpr (i < NU)
          return lds_read_async<((i & 1) ? kFrU + i / 2 : i / 2) * kFragElems * 2>(bn);
        else
          return lds_read_async<(i - NU) * kFragElems * 2>(bo);
      };
      u32x4 fr[DEPTH];
      static_for<0, DEPTH>([&](auto ic) {
        if constexpr (decltype(ic)::value < NF) fr[decltype(ic)::value] = read(ic);
      });
      u32x4 Z[2];
      float zl = 0.0f;
      auto gate = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const float z = silu_gate(Uc[k], Vc[k]);
        if constexpr (k % 2 == 0)
          zl = z;
        else
          Z[k / 8][(k % 8) / 2] = Ty::pack2(zl, z);
      };
      if constexpr (NO > 0 && NU == 0) static_for<0, 16>(gate);
      if constexpr (NU > 0) {
        Un = f32x16{};
        Vn = f32x16{};
      }
      static_for<0, NF>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr int after = NF - 1 - i < DEPTH - 1 ? NF - 1 - i : DEPTH - 1;
        lds_wait<after>(fr[i % DEPTH]);
        if constexpr (i < NU) {
          if constexpr (i % 2 == 0)
            Un = Ty::mma32(fr[i % DEPTH], Pu[i / 2], Un);
          else if constexpr (!F8)  // (stream runs only without F8)
            Vn = Ty::mma32(fr[i % DEPTH], Pv[i / 2], Vn);
        } else {
          constexpr int j = i - NU;
          W[j / 2] = Ty::mma32(Z[j % 2], fr[i % DEPTH], W[j / 2]);
        }
        if constexpr (i + DEPTH < NF) fr[i % DEPTH] = read(std::integral_constant<int, i + DEPTH>{});
        if constexpr (NO > 0 && i < NU) gate(ic);
      });
      if constexpr (NU > 0 && NO > 0) {
        static_for<0, NU>([&](auto) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x402, 6, 0);  // VALU, transcendental
        });
      }
    };
    using Nu = std::integral_constant<int, 2 * kKS>;
    using No = std::integral_constant<int, kFrO>;
    using Zero = std::integral_constant<int, 0>;
    auto base = [&](int ec) { return lds_addr(sh.w[ec % 3]) + lane16; };
    // Step ec waits for chunk ec + 1 (issued at step ec - 1, or before the loop for ec <= 1: at
    // ec = 0 chunk 2, issued after it, may still be in flight); the barrier also means every
    // wave is done with chunk ec - 1, whose buffer takes chunk ec + 2.
    // fp8: chunk ec + 1's U' (bf16 / f16) and V' (K = 64 e4m3) products, chunk ec's gate (V''s
    // dequantisation: f8_gate) and W += Z B_o, in stream8.
    const float deq8 = F8 ? f8_deq(a.packed) : 1.0f;
    // fp8 step as `stream`: the fragments read DEPTH8 ahead with untracked LDS reads in issue
    // order -- chunk en's 8 U' fragments, its 2 V' K = 64 fragments (two 16-byte halves each,
    // 32 bytes per lane), then chunk ec's 8 B_o fragments -- with two of chunk ec's gate values
    // after each U' product.  A V' fragment's halves are refilled together once both are used.
    constexpr int DEPTH8 = 4;
    auto stream8 = [&](auto hu_tag, auto ho_tag, int en, int ec, f32x16& Un, f32x16& Vn, const f32x16& Uc,
                       const f32x16& Vc) {
      constexpr bool HU = decltype(hu_tag)::value;  // chunk en's U' / V' products
      constexpr bool HO = decltype(ho_tag)::value;  // chunk ec's gate and W += Z B_o
      constexpr int NUR = HU ? kKS + 2 * KV : 0;    // reads of chunk en (8 U', 4 V' halves)
      constexpr int NF = NUR + (HO ? kFrO : 0);
      const uint32_t bu = HU ? lds_addr(sh.w[en % 3]) + lane16 : 0u;
      const uint32_t bv = HU ? lds_addr(sh.w[en % 3] + F8_BV * kFragElems) + 32u * static_cast<uint32_t>(lane) : 0u;
      const uint32_t bo = HO ? lds_addr(sh.w[ec % 3] + F8_BO * kFragElems) + lane16 : 0u;
      auto read = [&](auto ic) -> u32x4 {
        constexpr int i = decltype(ic)::value;
        if constexpr (i < kKS && HU)
          return lds_read_async<i * kFragElems * 2>(bu);
        else if constexpr (i < NUR)
          return lds_read_async<((i - kKS) / 2) * kF8K64Bytes + 16 * ((i - kKS) % 2)>(bv);
        else
          return lds_read_async<(i - NUR) * kFragElems * 2>(bo);
      };
      u32x4 fr[DEPTH8];
      static_for<0, DEPTH8>([&](auto ic) {
        if constexpr (decltype(ic)::value < NF) fr[decltype(ic)::value] = read(ic);
      });
      u32x4 Z[2];
      if constexpr (HU) {
        Un = f32x16{};
        Vn = f32x16{};
      }
      if constexpr (HO && !HU) {
#pragma unroll
        for (int k = 0; k < 16; k += 2)
          Z[k / 8][(k % 8) / 2] = Ty::pack2(f8_gate<Ty>(Uc[k], Vc[k], deq8), f8_gate<Ty>(Uc[k + 1], Vc[k + 1], deq8));
      }
      static_for<0, NF>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr bool FH = HU && i >= kKS && i < NUR && ((i - kKS) % 2) == 0;
        constexpr bool SH = HU && i >= kKS && i < NUR && ((i - kKS) % 2) == 1;
        // Reads issued after read i when iteration i waits: reads go out in index order, DEPTH8
        // at the start and one per finished read after (two after a V' second half).
        constexpr int younger = [] {
          int n = DEPTH8;
          for (int m = 0; m < i; ++m) {
            const bool fh = HU && m >= kKS && m < NUR && ((m - kKS) % 2) == 0;
            const bool sh2 = HU && m >= kKS && m < NUR && ((m - kKS) % 2) == 1;
            n += fh ? 0 : (sh2 ? 2 : 1);
          }
          n = n < NF ? n : NF;
          return n - 1 - i;
        }();
        constexpr int after = younger < 0 ? 0 : younger;
        lds_wait<after>(fr[i % DEPTH8]);
        if constexpr (HU && i < kKS) {
          Un = Ty::mma32(fr[i % DEPTH8], Pu[i], Un);
          if constexpr (HO) {
            constexpr int k = 2 * i;
            Z[k / 8][(k % 8) / 2] =
                Ty::pack2(f8_gate<Ty>(Uc[k], Vc[k], deq8), f8_gate<Ty>(Uc[k + 1], Vc[k + 1], deq8));
          }
        } else if constexpr (SH) {
          if constexpr (F8) {
            const u32x4 lo = fr[(i - 1) % DEPTH8], hi = fr[i % DEPTH8];
            const u32x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            Vn = mma32x64_f8(v8, Pv[(i - kKS) / 2], Vn);
          }
        } else if constexpr (i >= NUR) {
          constexpr int j = i - NUR;
          W[j / 2] = Ty::mma32(Z[j % 2], fr[i % DEPTH8], W[j / 2]);
        }
        // Refills: a read's slot takes the read DEPTH8 later once it is used (a V' first half
        // together with its second half).
        if constexpr (SH) {
          if constexpr (i - 1 + DEPTH8 < NF) fr[(i - 1) % DEPTH8] = read(std::integral_constant<int, i - 1 + DEPTH8>{});
          if constexpr (i + DEPTH8 < NF) fr[i % DEPTH8] = read(std::integral_constant<int, i + DEPTH8>{});
        } else if constexpr (!FH) {
          if constexpr (i + DEPTH8 < NF) fr[i % DEPTH8] = read(std::integral_constant<int, i + DEPTH8>{});
        }
      });
    };
    auto step = [&](int ec, f32x16& Uc, f32x16& Vc, f32x16& Un, f32x16& Vn) {
      const uint32_t bo = base(ec) + 2u * kFrU * kFragElems * 2u;
      if (ec + 1 < kNCH) {
        if (ec == 0)
          wait_chunk(E0{});
        else
          wait_lds_dma();
        __syncthreads();
        if (ec >= 1 && ec + 2 < kNCH) issue_chunk(ec + 2);
        if (act) {
          if constexpr (F8) {
            stream8(std::true_type{}, std::true_type{}, ec + 1, ec, Un, Vn, Uc, Vc);
          } else {
            stream(Nu{}, No{}, base(ec + 1), bo, Un, Vn, Uc, Vc);
          }
        }
      } else if (act) {
        if constexpr (F8)
          stream8(std::false_type{}, std::true_type{}, ec, ec, Un, Vn, Uc, Vc);
        else
          stream(Zero{}, No{}, 0u, bo, Un, Vn, Uc, Vc);
      }
    };
    f32x16 Ua, Va, Ub = {}, Vb = {};
    if (act) {
      if constexpr (F8)
        stream8(std::true_type{}, std::false_type{}, 0, 0, Ua, Va, Ub, Vb);
      else
        stream(Nu{}, Zero{}, base(0), 0u, Ua, Va, Ub, Vb);
    }
#pragma unroll
    for (int ec = 0; ec < kNCH; ec += 2) {
      step(ec, Ua, Va, Ub, Vb);
      step(ec + 1, Ub, Vb, Ua, Va);
    }

    // Output.  Past the barrier every wave is done with the chunk buffers: each stages its 32
    // rows of rounded delta (times the drop-path scale) there; the residual's x elements are
    // this unit's tile rows, read from LDS before the next unit's tile rows replace them.
    mfma_drain();
    __syncthreads();
    if (act) {
    const int piece = lane & 15;
    const int64_t colq = static_cast<int64_t>(qc) * kD;
    const u32x4 fAo = sh.tok_ops[2][lane];
    // delta^T: lane l32 = the wave's row l32, registers 4 q .. 4 q + 3 = channels 32 mb + 8 q +
    // 4 hh .. + 3, staged as 8-byte row pieces.
    f32x16 dl[kMB];
    pair_output_t<Ty, kMB>(W, fAo, lane, dl);
    mfma_drain();
    uint16_t* st = &sh.w[0][0] + wave * 32 * kLdo;
    const float sc = sh.dsc[s][2 * wave + ((lane >> 4) & 1)];
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t v0 = Ty::pack2(dl[mb][4 * q], dl[mb][4 * q + 1]);
        uint32_t v1 = Ty::pack2(dl[mb][4 * q + 2], dl[mb][4 * q + 3]);
        if (a.drop_scale) {
          v0 = Ty::pack2(Ty::to_f32(lo16(v0)) * sc, Ty::to_f32(hi16(v0)) * sc);
          v1 = Ty::pack2(Ty::to_f32(lo16(v1)) * sc, Ty::to_f32(hi16(v1)) * sc);
        }
        *reinterpret_cast<u32x2*>(&st[l32 * kLdo + 32 * mb + 8 * q + 4 * hh]) = u32x2{v0, v1};
      }
    // Pass k covers piece lane % 16 of rows lane / 16 + 4 k of the wave (tile slot of the piece:
    // piece ^ tile128_swz(row)).
    u32x4 xv[8], val[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int rr = (lane >> 4) + 4 * k;
      xv[k] = *reinterpret_cast<const u32x4*>(&sh.x[(32 * wave + rr) * kD + ((piece ^ tile128_swz(rr)) * 8)]);
    }
    wave_lds_sync();
#pragma unroll
    for (int k = 0; k < 8; ++k) val[k] = *reinterpret_cast<const u32x4*>(&st[((lane >> 4) + 4 * k) * kLdo + piece * 8]);
    // The tile reads are complete (their values are in registers): the next unit's rows go out
    // (strided groups: fetched through registers after the stores).
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (QW == 0) {
      if (has_next) issue_tile(s ^ 1);
    }
    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(a.out, xbytes);
    const __amdgpu_buffer_rsrc_t rs =
        buffer_rsrc(a.stats_out, static_cast<uint32_t>(static_cast<int64_t>(a.batch) * a.n_tok * a.q_c * 4));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int rr = (lane >> 4) + 4 * k;
      const int32_t id = sh.rowout[s][32 * wave + rr];
      u32x4 v = val[k];
      if (a.residual) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = add_residual2<Ty>(xv[k][e], v[e]);
      }
      if (a.stats_out) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(v[e], acc);
        acc = group_sum<16>(acc);
        const uint32_t so = (piece == 15 && id >= 0) ? (static_cast<uint32_t>(id) * a.q_c + qc) * 4u : kOffOut;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc), rs, so, 0, 0);
      }
      if constexpr (NS == 1) {
        const uint32_t oo = id >= 0 ? static_cast<uint32_t>(id) * static_cast<uint32_t>(a.channels * 2) +
                                          static_cast<uint32_t>(colq * 2) + 16u * piece
                                    : kOffOut;
        __builtin_amdgcn_raw_buffer_store_b128(v, ro, oo, 0, 0);
      } else {
        *reinterpret_cast<u32x4*>(&st[((lane >> 4) + 4 * k) * kLdo + piece * 8]) = v;  // final values
      }
    }
    if constexpr (NS > 1) {
      // Strided groups: tile column t is channel res + t NS of the row; lane l stores column
      // 64 h + l of one row per instruction, so the lanes writing one 128-byte line of out come
      // together in one request (2-byte elements: the other groups' columns lie in between).
      wave_lds_sync();
#pragma unroll 4
      for (int rr = 0; rr < 32; ++rr) {
        const int32_t id = sh.rowout[s][32 * wave + rr];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int t = 64 * h + lane;
          const uint16_t v = st[rr * kLdo + t];
          const uint32_t ob = id >= 0 ? static_cast<uint32_t>(id) * static_cast<uint32_t>(a.channels * 2) +
                                            2u * static_cast<uint32_t>(res_g + t * NS)
                                      : kOffOut;
          __builtin_amdgcn_raw_buffer_store_b16(v, ro, ob, 0, 0);
        }
      }
    }
    } else if constexpr (QW == 0) {
      if (has_next) issue_tile(s ^ 1);
    }
    if constexpr (QW > 0) {
      if (has_next) {
        TileBatch vpre;
        tile_fetch(s ^ 1, 0, vpre);
        strided_tile(s ^ 1, vpre);
      }
    }
    if (has_next) {
      stats_write(snext, id_next, s ^ 1);
      wave_lds_sync();
      __syncthreads();  // every wave is done with its staging rows, which chunk 0 overwrites
      issue_chunk(0);
      // The next unit's tile rows have landed once at most this unit's stores (8 row pieces, 8
      // statistics values) and chunk 0's copies, all issued after them, are outstanding
      // (strided groups: the rows were written by this wave).
      if constexpr (QW == 0) {
        if (a.stats_out)
          wait_chunk(std::integral_constant<int, 16>{});
        else
          wait_chunk(std::integral_constant<int, 8>{});
      }
    }
  }
}

}  // namespace

bool persist_supported(int32_t d, int32_t rd, int32_t channels, int32_t q_c, int64_t x_elems) {
  return d == kD && rd == kRD && channels == q_c * kD && x_elems * 2 < (int64_t(1) << 31);
}

template <class Ty>
void launch_stride(const PersistArgs& a, dim3 g, int32_t n, int32_t n_pairs, hipStream_t stream) {
  auto go = [&](auto f8_tag, auto ns_tag) {
    constexpr bool F8 = decltype(f8_tag)::value;
    constexpr int NS = decltype(ns_tag)::value;
    hipLaunchKernelGGL((bigemm_fwd_persist_kernel<Ty, F8, NS>), g, dim3(kThreads), 0, stream, a, n, n_pairs);
  };
  auto by_ns = [&](auto f8_tag) {
    switch (a.stride) {
      case 2: go(f8_tag, std::integral_constant<int, 2>{}); break;
      case 4: go(f8_tag, std::integral_constant<int, 4>{}); break;
      case 8: go(f8_tag, std::integral_constant<int, 8>{}); break;
      default: go(f8_tag, std::integral_constant<int, 1>{}); break;
    }
  };
  if (a.fp8)
    by_ns(std::true_type{});
  else
    by_ns(std::false_type{});
}

int launch_fwd_persist(const PersistArgs& a, int32_t dtype, hipStream_t stream) {
  const int64_t chunks = (static_cast<int64_t>(a.batch) * a.q_s + kGroups - 1) / kGroups;
  const int64_t units = chunks * a.q_c;
  if (units == 0) return OW_OK;
  if (units > 0x7fffffff) return fail(OW_ERR_UNSUPPORTED, "grid too large (%lld units)", (long long)units);
  // With at most one unit per CU, one workgroup per unit.  With more, one workgroup per CU, the
  // grid a multiple of 8 (whole XCD rounds) and of q_c.  Contiguous groups: whole units round
  // robin (workgroup b, and so its XCD, keeps group b % q_c).  Strided groups: each group's
  // pairs split evenly over its grid / q_c workgroups, so that the last round's 2-byte stores
  // come from all 8 XCDs (at 416 units on 256 CUs, 14x14x512 batch 128, a round robin left the
  // second round on 5 of them) and from partial units whose idle waves store nothing.
  const int64_t cus = device_cus();
  int64_t grid = units;
  int32_t n_pairs = 0;
  if (cus < units) {
    int64_t m = 8;
    while (m % a.q_c) m += 8;  // lcm(8, q_c)
    grid = cus - cus % m;
    if (grid < m) grid = m;
    n_pairs = a.stride > 1 ? static_cast<int32_t>((static_cast<int64_t>(a.batch) * a.q_s + 1) / 2) : -1;
  }
  const dim3 g(static_cast<unsigned>(grid));
  if (a.norm == kNormInline && a.stride == 1)
    return fail(OW_ERR_INVALID, "the persistent forward with contiguous groups takes precomputed row statistics");
  if (a.fp8 && a.norm == kNormNone) return fail(OW_ERR_INVALID, "the fp8 channel side needs the fused RMSNorm");
  const int32_t n = static_cast<int32_t>(units);
  if (dtype != OW_DTYPE_BF16 && dtype != OW_DTYPE_F16) return fail(OW_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (a.stride != 1 && a.stride != 2 && a.stride != 4 && a.stride != 8)
    return fail(OW_ERR_UNSUPPORTED, "persistent forward: channel stride %d", a.stride);
  if (a.stride != 1 && a.stride != a.q_c) return fail(OW_ERR_INVALID, "strided groups need stride == q_c");
  if (dtype == OW_DTYPE_BF16)
    launch_stride<BF16>(a, g, n, n_pairs, stream);
  else
    launch_stride<F16>(a, g, n, n_pairs, stream);
  return hip_status(hipGetLastError(), "bigemm_fwd_persist_kernel launch");
}

}  // namespace ow
