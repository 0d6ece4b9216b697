// Device-side helpers shared by the BiGEMM kernels: vector types, per-dtype traits (rounding,
// packing, MFMA), the reference's RMSNorm dtype sequence and the folded SiLU gate.
//
// MFMA layouts (64 lanes; l16 = lane % 16, h = lane / 16, l32 = lane % 32, hh = lane / 32):
//   16x16 accumulator        lane holds D[4h + i][l16], i = 0..3
//   16x16x16 A / B operand   lane holds A[l16][4h + j] / B[4h + j][l16], j = 0..3
//   32x32 accumulator        lane holds D[8(i/4) + 4hh + i%4][l32], i = 0..15
//   32x32x16 A / B operand   lane holds 8 K-slots j = 0..7 of row / column l32 for K half hh
// Only the pairing of A slot (hh, j) with B slot (hh, j) is fixed by the hardware, so each
// operand may use any K order as long as both sides agree.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "ow_common.h"

namespace ow {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kG = 16;                      // spatial tile (tokens per group)
constexpr int kFragElems = 512;             // 32x32x16 operand: 64 lanes x 8
constexpr int kHeadElems = 3 * kFragElems;  // token-side operands (A_u, A_v, A_o rows) at the head of the packed weights
constexpr float kNegLog2e = -1.4426950408889634f;
constexpr float kNegLn2 = -0.6931471805599453f;

__device__ __forceinline__ uint16_t lo16(uint32_t v) { return static_cast<uint16_t>(v & 0xffffu); }
__device__ __forceinline__ uint16_t hi16(uint32_t v) { return static_cast<uint16_t>(v >> 16); }

// A constant in a scalar register that the compiler cannot fold into an instruction's constant
// operand (the asm is not volatile, so it is still hoisted and shared).
__device__ __forceinline__ uint32_t opaque_sgpr(uint32_t c) {
  uint32_t r;
  asm("; opaque constant %0" : "=s"(r) : "0"(c));
  return r;
}

struct BF16 {
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  static __device__ __forceinline__ float to_f32(uint16_t u) {
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  // a.lo^2 + a.hi^2 + acc in fp32
  static __device__ __forceinline__ float dot2sq(uint32_t a, float acc) {
    const bf16x2 v = __builtin_bit_cast(bf16x2, a);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
  }
  // x.lo + v.lo (H = 0) or x.hi + v.hi (H = 1) in fp32 with one rounding: a dot product of v with
  // (1, 0) or (0, 1) accumulated onto the widened half of x (the products are exact).  The
  // selector goes through a scalar register (opaque_sgpr): as a literal the compiler encodes
  // (1, 0) as the inline constant 1.0, which this instruction does not read as (1, 0).
  template <int H>
  static __device__ __forceinline__ float add_half(uint32_t x, uint32_t v) {
    const bf16x2 sel = __builtin_bit_cast(bf16x2, opaque_sgpr(H ? 0x3f800000u : 0x00003f80u));
    return __builtin_amdgcn_fdot2_f32_bf16(sel, __builtin_bit_cast(bf16x2, v), to_f32(H ? hi16(x) : lo16(x)), false);
  }
  static __device__ __forceinline__ f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                     __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16k32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  }
};

struct F16 {
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  static __device__ __forceinline__ float to_f32(uint16_t u) {
    return static_cast<float>(__builtin_bit_cast(_Float16, u));
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  static __device__ __forceinline__ float dot2sq(uint32_t a, float acc) {
    const f16x2 v = __builtin_bit_cast(f16x2, a);
    return __builtin_amdgcn_fdot2(v, v, acc, false);
  }
  template <int H>
  static __device__ __forceinline__ float add_half(uint32_t x, uint32_t v) {
    const f16x2 sel = __builtin_bit_cast(f16x2, opaque_sgpr(H ? 0x3c000000u : 0x00003c00u));
    return __builtin_amdgcn_fdot2(sel, __builtin_bit_cast(f16x2, v), to_f32(H ? hi16(x) : lo16(x)), false);
  }
  static __device__ __forceinline__ f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16k32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  }
};

template <class Ty>
__device__ __forceinline__ float round_to(float f) {
  return Ty::to_f32(Ty::from_f32(f));
}

// RMSNorm row scale with the reference's dtype sequence (omniweave/models/block.py:83-84):
// var (fp32) -> x.dtype, + eps in x.dtype, rsqrt in x.dtype.
template <class Ty>
__device__ __forceinline__ float rms_scale(float mean_sq, float eps) {
  const float v = round_to<Ty>(round_to<Ty>(mean_sq) + eps);
  return round_to<Ty>(rsqrtf(v));
}

// SiLU(U) V from the folded accumulators U' = -log2(e) U, V' = -ln(2) V:
// SiLU(U) V = U V / (1 + e^-U) = U' V' / (1 + 2^U').
__device__ __forceinline__ float silu_gate(float up, float vp) {
  return up * vp * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(up));
}

// Separates MFMA results from VALU reads of them by 32 wait states.  Used where the read
// follows the MFMA across a basic-block boundary (loop exit), or where many accumulator
// registers are read at once: the hardware does not interlock an MFMA's result against a
// later VALU read, and a read a few instructions after a 16x16x16 MFMA returns the old value
// of its last accumulator register.  The scheduling barriers keep the compiler from moving
// MFMAs or reads across the padding.
__device__ __forceinline__ void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Makes this wave's LDS writes visible to its other lanes before they read them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}


// round(x + v) on two packed values (low and high halves): the residual of the block output,
// x the input and v the rounded delta.
//
// Each half is one 2-element dot product of v with (1, 0) or (0, 1) accumulated onto the widened
// half of x: the products are exact, so the fp32 result is the rounded sum x + v, as a separate
// fp32 add forms it (only signed zeros may differ: -0 + -0 can give +0).  Two instructions per
// value instead of an unpack of each operand and an add.
template <class Ty>
__device__ __forceinline__ uint32_t add_residual2(uint32_t x, uint32_t v) {
  return Ty::pack2(Ty::template add_half<0>(x, v), Ty::template add_half<1>(x, v));
}

// Direct global -> LDS copy of one 1 KB operand fragment by one wave (16 bytes per lane, LDS
// address M0 + 16 lane).  Issued as inline assembly so that the compiler does not track it: for
// the builtin it waits for every outstanding LDS DMA before the next LDS read, which would
// serialise each weight chunk's copy with the reads of the chunk before it.  The kernel waits
// for the copies itself (wait_vmcnt / wait_lds_dma) before the barrier that publishes a chunk,
// and nothing else in the kernel uses M0.
// src and dst are wave-uniform (scalar base address, M0); the lane's byte offset lane16 = 16 lane
// is the only vector operand.
// lds: LDS byte address of the destination.
__device__ __forceinline__ void copy_frag_to_lds_at(const uint16_t* src, uint32_t lds, uint32_t lane16) {
  lds = __builtin_amdgcn_readfirstlane(lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(lane16), "s"(src), "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}
__device__ __forceinline__ void copy_frag_to_lds(const uint16_t* src, uint16_t* dst, uint32_t lane16) {
  copy_frag_to_lds_at(src, static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)dst)),
                      lane16);
}

// Raw buffer resource over `bytes` bytes at p (no stride): loads past the end return zero and
// stores there are dropped, so pad rows need no branches (callers keep buffers below 2 GiB).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
constexpr uint32_t kOffOut = 0x80000000u;  // a byte offset past every buffer below 2 GiB

// 16 bytes per lane from a buffer (byte offset voff, kOffOut: zeros) to LDS byte address
// lds + 16 lane (lds wave-uniform), untracked by the compiler (no compiler wait before later LDS
// reads); the kernel waits with wait_vmcnt.
__device__ __forceinline__ void tile_copy(__amdgpu_buffer_rsrc_t rx, uint32_t voff, uint32_t lds) {
  lds = __builtin_amdgcn_readfirstlane(lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rx),
               "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}
// The same with the non-temporal cache policy, for data read exactly once.
__device__ __forceinline__ void tile_copy_nt(__amdgpu_buffer_rsrc_t rx, uint32_t voff, uint32_t lds) {
  lds = __builtin_amdgcn_readfirstlane(lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds" ::"v"(voff), "s"(rx),
               "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// A wave-uniform pointer the compiler may not prove uniform (the scalar operand of a copy).
__device__ __forceinline__ const uint16_t* uniform_ptr(const uint16_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint16_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ void wait_lds_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Waits until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// ds_read_b128 at byte offset OFF from addr, issued as inline assembly: the compiler neither
// moves it next to its use nor waits for it, so several reads stay in flight.  Under the d = 128
// kernel's register pressure the compiler otherwise keeps a single fragment register and waits
// for every read right before its MFMA.  The value is used only after lds_wait<N>(v), N = the
// number of LDS reads issued after this one: LDS returns in order, so LDS or scalar-memory
// operations of the compiler issued in between can only make that wait stricter.
template <int OFF>
__device__ __forceinline__ u32x4 lds_read_async(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x4& v) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// The M = 8/n elements of a strided channel group held by one 16-byte row vector (element
// index res + t n for t < M, res < n the group's first channel), packed in order: M = 4 and
// M = 2 as 16-bit halves of two / one word, M = 1 in the low half.  res is wave-uniform, so
// the word choices are uniform selects and each pair of halves is one v_perm_b32 (result
// bytes 0-1 from the low operand, 2-3 from the high one).
template <int M>
using StridedPack = std::conditional_t<M == 4, u32x2, uint32_t>;

template <int M>
__device__ __forceinline__ StridedPack<M> strided_pack(const u32x4& v, int res) {
  const uint32_t sel = (res & 1) ? 0x07060302u : 0x05040100u;  // high or low halves
  if constexpr (M == 4) {  // n = 2: halves (res & 1) of words 0..3
    return u32x2{__builtin_amdgcn_perm(v[1], v[0], sel), __builtin_amdgcn_perm(v[3], v[2], sel)};
  } else if constexpr (M == 2) {  // n = 4: words res / 2 and res / 2 + 2
    const bool w1 = (res & 2) != 0;
    return __builtin_amdgcn_perm(w1 ? v[3] : v[2], w1 ? v[1] : v[0], sel);
  } else {  // n = 8: word res / 2
    const int w = res >> 1;
    const uint32_t word = w == 0 ? v[0] : w == 1 ? v[1] : w == 2 ? v[2] : v[3];
    return (res & 1) ? word >> 16 : word;
  }
}

// ---------------------------------------------------------------------------------------
// One 32-token pair (token groups 0 and 1 of 16 tokens) of a channel group, all on 32x32x16
// MFMAs.  Token-side products use the block-diagonal 32x32 token matrix: K step g covers the
// 16 tokens of group g, and lanes whose token (lane % 32) is in the other group get a zero B
// operand for that step.  Token order within a K step: slot j of lane half hh is token
// kord(j, hh) = 8(j/4) + 4hh + j%4, the row order of a 32x32 accumulator, so the x values a lane
// reads for the token side are the ones its output accumulator needs for the residual.
//
//   P^T  = X^T (A diag r)^T     A operand X^T: lane (c = l32, hh) slot j = x[16g + kord(j, hh)][c]
//                               B operand:     lane (t = l32, hh) slot j = A[t % 16][kord(j, hh)] r[16g + kord(j, hh)]
//        accumulator lane (t, hh) register i = channel kord(i) of the 32-channel block, so
//        registers 8s..8s+7 are K step s of the next product with channel order
//        16 ks + kord(j, hh) (the packed B_u'^T / B_v'^T use that order)
//   U'^T = B_u'^T P_u^T         accumulator lane (t, hh) register i = expanded row kord(i)
//   W    = Z B_o                A operand Z (lane = token), B operand B_o (lane = channel), K order
//                               of the expanded dim as held by the U'^T accumulator;
//        accumulator lane (c = l32, hh) register i = token kord(i)
//   delta = A_o W               A operand: lane (t, hh) slot j = A_o[t % 16][kord(j, hh)] for
//                               K step g = t / 16 (zero otherwise), B operand = W registers
//        accumulator lane (c, hh) register i = delta[token kord(i)][channel c], where register
//        8g + j is token 16g + kord(j, hh): slot j of the lane's X^T operand for K step g

__device__ __forceinline__ int pair_token_row(int i, int hh) { return 8 * (i >> 2) + 4 * hh + (i & 3); }

// X^T operand: rows p[k ld] for k = 0..3, 8..11 of one LDS column (p = row 16g + 4hh).  Each
// 32-bit word is filled half by half (16-bit loads into the low / high half of a register).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 column8(const uint16_t* p, int ld) {
  u32x4 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k0 = 8 * (q >> 1) + 2 * (q & 1);
    u16x2 w;
    w.x = p[k0 * ld];
    w.y = p[(k0 + 1) * ld];
    v[q] = __builtin_bit_cast(uint32_t, w);
  }
  return v;
}

// Sum over aligned groups of N lanes (N in {8, 16, 32}) with DPP; the total lands in the last
// lane of each group (lane % N == N - 1), the other lanes hold partial sums.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}

template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 8 || N == 16 || N == 32, "group of 8, 16 or 32 lanes");
  v += dpp_f32<0xb1, 0xf>(v);                          // quad_perm 1,0,3,2
  v += dpp_f32<0x4e, 0xf>(v);                          // quad_perm 2,3,0,1
  v += dpp_f32<0x141, 0xf>(v);                         // row_half_mirror: quads of 8 lanes
  if constexpr (N >= 16) v += dpp_f32<0x140, 0xf>(v);  // row_mirror: halves of a 16-lane row
  if constexpr (N == 32) v += dpp_f32<0x142, 0xa>(v);  // row_bcast15: row 2k into row 2k + 1
  return v;
}

// Token-operand row (8 values, packed, slot j <-> token kord(j, hh)) scaled by the RMSNorm
// scales of those tokens; r points at the scale of token 16g + 4hh.
template <class Ty>
__device__ __forceinline__ u32x4 scale8(u32x4 a, const float* r) {
  u32x4 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k0 = 8 * (q >> 1) + 2 * (q & 1);
    v[q] = Ty::pack2(Ty::to_f32(lo16(a[q])) * r[k0], Ty::to_f32(hi16(a[q])) * r[k0 + 1]);
  }
  return v;
}

__device__ __forceinline__ u32x4 keep_if(bool keep, u32x4 v) {
  return keep ? v : u32x4{0u, 0u, 0u, 0u};
}

// Accumulator registers 8s..8s+7 as a packed K step.
template <class Ty>
__device__ __forceinline__ u32x4 pack_kstep(const f32x16& acc, int s) {
  return u32x4{Ty::pack2(acc[8 * s + 0], acc[8 * s + 1]), Ty::pack2(acc[8 * s + 2], acc[8 * s + 3]),
               Ty::pack2(acc[8 * s + 4], acc[8 * s + 5]), Ty::pack2(acc[8 * s + 6], acc[8 * s + 7])};
}

// Token side of a pair: Pu/Pv[ks] (ks < KS) from the pair's 32 LDS rows `tl` (row stride ld).
// col[cb] is the LDS column holding channel 32 cb + l32 of the group; bu/bv are the lane's
// (already r-scaled) token-operand rows, used for the K step of the lane's own group.  The X^T
// operands read are returned in xk[cb][g] (the residual of the lane's output elements).
template <class Ty, int KS>
__device__ __forceinline__ void pair_token_side_mma(const u32x4 (&xk)[KS / 2][2], u32x4 bu, u32x4 bv, int lane,
                                                    u32x4 (&Pu)[KS], u32x4 (&Pv)[KS]) {
  const bool g0 = (lane & 16) == 0;
  const u32x4 bu0 = keep_if(g0, bu), bu1 = keep_if(!g0, bu);
  const u32x4 bv0 = keep_if(g0, bv), bv1 = keep_if(!g0, bv);
  const f32x16 zero = {};
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    const u32x4 x0 = xk[cb][0], x1 = xk[cb][1];
    f32x16 pu = Ty::mma32(x0, bu0, zero);
    f32x16 pv = Ty::mma32(x0, bv0, zero);
    pu = Ty::mma32(x1, bu1, pu);
    pv = Ty::mma32(x1, bv1, pv);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      Pu[2 * cb + s] = pack_kstep<Ty>(pu, s);
      Pv[2 * cb + s] = pack_kstep<Ty>(pv, s);
    }
  }
}

// 16-byte piece swizzle of a [rows][128] 16-bit tile (256-byte rows): piece p of row r sits at
// slot p ^ tile128_swz(r).  The four rows that a 16-lane transposed read (pair_xt_tr) or a 1 KB
// copy covers then fall in four different 64-byte bank windows.
__device__ __forceinline__ int tile128_swz(int r) { return 4 * (r & 3); }

// X^T operands of a pair (as pair_token_side reads them) by transposed LDS reads
// (ds_read_b64_tr_b16): in each group of 16 lanes, lane L reads the 8 bytes of row r0 + L / 4 at
// channel c0 + 4 (L % 4), and lane i of the group then holds channel c0 + i of rows r0 .. r0 + 3
// (element k = row r0 + k).  Lane (l32, hh) needs rows 16 g + 4 hh + 0..3 and 16 g + 8 + 4 hh +
// 0..3 of channel 32 cb + l32: two reads per operand instead of eight 16-bit reads.  at(r, c)
// is the LDS byte address of pair row r, channel c (4 consecutive channels must be adjacent).
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_read_tr16(uint32_t addr) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_s16x4*>(static_cast<uintptr_t>(addr)));
  return __builtin_bit_cast(u32x2, v);
}
template <int KS, class At>
__device__ __forceinline__ void pair_xt_tr(At at, int lane, u32x4 (&xk)[KS / 2][2]) {
  const int hh = lane >> 5, l16 = lane & 15, half = (lane >> 4) & 1;
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    const int c = 32 * cb + 16 * half + 4 * (l16 & 3);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int r = 16 * g + 4 * hh + (l16 >> 2);
      const u32x2 a = lds_read_tr16(at(r, c)), b = lds_read_tr16(at(r + 8, c));
      xk[cb][g] = u32x4{a[0], a[1], b[0], b[1]};
    }
  }
}

template <class Ty, int KS>
__device__ __forceinline__ void pair_token_side(const uint16_t* tl, int ld, const int (&col)[KS / 2], u32x4 bu,
                                                u32x4 bv, int lane, u32x4 (&Pu)[KS], u32x4 (&Pv)[KS],
                                                u32x4 (&xk)[KS / 2][2]) {
  const int hh = lane >> 5;
  const bool g0 = (lane & 16) == 0;
  const u32x4 bu0 = keep_if(g0, bu), bu1 = keep_if(!g0, bu);
  const u32x4 bv0 = keep_if(g0, bv), bv1 = keep_if(!g0, bv);
  const f32x16 zero = {};
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    xk[cb][0] = column8(tl + (4 * hh) * ld + col[cb], ld);
    xk[cb][1] = column8(tl + (16 + 4 * hh) * ld + col[cb], ld);
  }
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    const u32x4 x0 = xk[cb][0], x1 = xk[cb][1];
    f32x16 pu = Ty::mma32(x0, bu0, zero);
    f32x16 pv = Ty::mma32(x0, bv0, zero);
    pu = Ty::mma32(x1, bu1, pu);
    pv = Ty::mma32(x1, bv1, pv);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      Pu[2 * cb + s] = pack_kstep<Ty>(pu, s);
      Pv[2 * cb + s] = pack_kstep<Ty>(pv, s);
    }
  }
}

// One 32-row chunk of the expanded dimension: U'^T, V'^T from the chunk's B_u'^T / B_v'^T
// fragments, Z = U'V' / (1 + 2^U'), W[mb] += Z B_o.  fu(ks), fv(ks), fo(mb, s) return fragments.
template <class Ty, int KS, int MB, class FU, class FV, class FO>
__device__ __forceinline__ void pair_chunk(const u32x4 (&Pu)[KS], const u32x4 (&Pv)[KS], FU fu, FV fv, FO fo,
                                           f32x16 (&W)[MB]) {
  f32x16 U = {}, V = {};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    U = Ty::mma32(fu(ks), Pu[ks], U);
    V = Ty::mma32(fv(ks), Pv[ks], V);
  }
  u32x4 Z[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      Z[s][q] = Ty::pack2(silu_gate(U[8 * s + 2 * q], V[8 * s + 2 * q]),
                          silu_gate(U[8 * s + 2 * q + 1], V[8 * s + 2 * q + 1]));
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int s = 0; s < 2; ++s) W[mb] = Ty::mma32(Z[s], fo(mb, s), W[mb]);
}

// ---- fp8 (OCP e4m3fn) channel side ----------------------------------------------------------
// Only V' = P_v B_v'' runs on fp8: with e4m3's 3-bit mantissa every quantised operand adds
// ~2.6% rel-L2 and the four of U' and V' together put delta ~5.4% from fp32, past the 5e-2
// gate, while one side alone stays near 3.8%.  V' uses the double-rate K = 64 MFMA
// (v_mfma_f32_32x32x64_f8f6f4): per 32-row chunk of the expanded dimension, d / 64 products
// instead of d / 16.
//
// Byte layout of an fp8 packed buffer: the Ty token-side head (kHeadElems elements), then
// kF8ScaleFloats floats of scales, then per (q, 32-row chunk ec), in 1 KB units: KS Ty B_u'^T
// fragments (as the Ty layout), d / 64 fp8 B_v'^T K64 fragments (2 KB: 64 lanes x 32 bytes)
// and 2 MB Ty B_o fragments, the chunk padded to a multiple of 4 units (whole copy rounds of
// 4 waves).  The dequantisation factor of V' is folded into the packed B_o (Z is linear in
// V'), the quantisation multiplier of P_v into the token operand A_v diag(r).
constexpr int kF8K64Bytes = 2048;
constexpr int kF8ScaleFloats = 16;
constexpr int kF8HeadBytes = kHeadElems * 2 + kF8ScaleFloats * 4;
// Scale slots: V' dequantisation (folded into B_o by the packer), P_v quantisation multiplier
// (448 / bound of |P_v|), absmax of the folded B_v''.
constexpr int kF8DeqV = 0, kF8QuantPv = 1, kF8AmaxBv = 2;
constexpr float kF8Max = 448.0f;

// Gate of the fp8 channel side from U' and the quantised V' (ow_pack_weights_fp8): with bf16
// activations V''s dequantisation factor is folded into the packed B_o (Z = SiLU(U) V stays in
// the quantised scale, far inside bf16 range); with f16 activations that Z would overflow f16
// (|V'| reaches 1e4 - 1e5), so the factor deq is applied here and the packed B_o carries none.
template <class Ty>
__device__ __forceinline__ float f8_gate(float up, float vq, float deq) {
  if constexpr (std::is_same_v<Ty, F16>)
    return silu_gate(up, vq * deq);
  else
    return silu_gate(up, vq);
}
// V''s dequantisation factor from an fp8 packed buffer (its scale slots follow the head).
__device__ __forceinline__ float f8_deq(const uint16_t* packed) {
  return reinterpret_cast<const float*>(packed + kHeadElems)[kF8DeqV];
}

// 1 KB units of one fp8 chunk for channel tile d.
__host__ __device__ constexpr int f8_chunk_units(int d) {
  return ((d / 16 + 2 * (d / 64) + 2 * (d / 32)) + 3) / 4 * 4;
}

typedef unsigned int u32x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

// Two floats -> two e4m3fn bytes (round to nearest even) in the low (HI = false) or high half
// of `old`.
template <bool HI>
__device__ __forceinline__ uint32_t cvt_fp8x2(float a, float b, uint32_t old) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, static_cast<int>(old), HI));
}

// K64 fp8 operand from the P^T accumulators of two 32-channel blocks (b0: channels 0..31 of the
// K step, b1: 32..63): slot j < 16 is register j of b0, slot j >= 16 register j - 16 of b1, so
// lane (t, hh) slot j holds channel 32 (j / 16) + 8 ((j % 16) / 4) + 4 hh + j % 4 of token t.
__device__ __forceinline__ u32x8 pack_k64_f8(const f32x16& b0, const f32x16& b1) {
  u32x8 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[q] = cvt_fp8x2<true>(b0[4 * q + 2], b0[4 * q + 3], cvt_fp8x2<false>(b0[4 * q], b0[4 * q + 1], 0u));
    v[4 + q] = cvt_fp8x2<true>(b1[4 * q + 2], b1[4 * q + 3], cvt_fp8x2<false>(b1[4 * q], b1[4 * q + 1], 0u));
  }
  return v;
}

// 32x32x64 e4m3 x e4m3 -> fp32 (no block scales).
__device__ __forceinline__ f32x16 mma32x64_f8(u32x8 a, u32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(__builtin_bit_cast(i32x8, a), __builtin_bit_cast(i32x8, b), c,
                                                          0, 0, 0, 0, 0, 0);
}

// Token-operand row scaled by the RMSNorm scales times m (see scale8).
template <class Ty>
__device__ __forceinline__ u32x4 scale8m(u32x4 a, const float* r, float m) {
  u32x4 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k0 = 8 * (q >> 1) + 2 * (q & 1);
    v[q] = Ty::pack2(Ty::to_f32(lo16(a[q])) * (r[k0] * m), Ty::to_f32(hi16(a[q])) * (r[k0 + 1] * m));
  }
  return v;
}

// Token side of a pair for the fp8 variant: P_u as Ty K steps (pair_token_side), P_v (whose
// token operand bv already carries the quantisation multiplier) as fp8 K64 operands.
template <class Ty, int KS>
__device__ __forceinline__ void pair_token_side_f8(const uint16_t* tl, int ld, const int (&col)[KS / 2], u32x4 bu,
                                                   u32x4 bv, int lane, u32x4 (&Pu)[KS], u32x8 (&Pv)[KS / 4],
                                                   u32x4 (&xk)[KS / 2][2]) {
  const int hh = lane >> 5;
  const bool g0 = (lane & 16) == 0;
  const u32x4 bu0 = keep_if(g0, bu), bu1 = keep_if(!g0, bu);
  const u32x4 bv0 = keep_if(g0, bv), bv1 = keep_if(!g0, bv);
  const f32x16 zero = {};
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    xk[cb][0] = column8(tl + (4 * hh) * ld + col[cb], ld);
    xk[cb][1] = column8(tl + (16 + 4 * hh) * ld + col[cb], ld);
  }
  f32x16 pv_prev = zero;
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    const u32x4 x0 = xk[cb][0], x1 = xk[cb][1];
    f32x16 pu = Ty::mma32(x0, bu0, zero);
    f32x16 pv = Ty::mma32(x0, bv0, zero);
    pu = Ty::mma32(x1, bu1, pu);
    pv = Ty::mma32(x1, bv1, pv);
#pragma unroll
    for (int s = 0; s < 2; ++s) Pu[2 * cb + s] = pack_kstep<Ty>(pu, s);
    if (cb & 1)
      Pv[cb / 2] = pack_k64_f8(pv_prev, pv);
    else
      pv_prev = pv;
  }
}

// pair_token_side_f8 from X^T operands already read (pair_xt_tr).
template <class Ty, int KS>
__device__ __forceinline__ void pair_token_side_f8_mma(const u32x4 (&xk)[KS / 2][2], u32x4 bu, u32x4 bv, int lane,
                                                       u32x4 (&Pu)[KS], u32x8 (&Pv)[KS / 4]) {
  const bool g0 = (lane & 16) == 0;
  const u32x4 bu0 = keep_if(g0, bu), bu1 = keep_if(!g0, bu);
  const u32x4 bv0 = keep_if(g0, bv), bv1 = keep_if(!g0, bv);
  const f32x16 zero = {};
  f32x16 pv_prev = zero;
#pragma unroll
  for (int cb = 0; cb < KS / 2; ++cb) {
    const u32x4 x0 = xk[cb][0], x1 = xk[cb][1];
    f32x16 pu = Ty::mma32(x0, bu0, zero);
    f32x16 pv = Ty::mma32(x0, bv0, zero);
    pu = Ty::mma32(x1, bu1, pu);
    pv = Ty::mma32(x1, bv1, pv);
#pragma unroll
    for (int s = 0; s < 2; ++s) Pu[2 * cb + s] = pack_kstep<Ty>(pu, s);
    if (cb & 1)
      Pv[cb / 2] = pack_k64_f8(pv_prev, pv);
    else
      pv_prev = pv;
  }
}

// pair_chunk for the fp8 variant: U' on Ty MFMAs, V' on K64 fp8 MFMAs (fv(s) returns the
// chunk's fp8 B_v'^T K64 fragment s), the gate (f8_gate) and Z B_o as pair_chunk.
template <class Ty, int KS, int MB, class FU, class FV, class FO>
__device__ __forceinline__ void pair_chunk_f8(const u32x4 (&Pu)[KS], const u32x8 (&Pv)[KS / 4], FU fu, FV fv, FO fo,
                                              f32x16 (&W)[MB], float deq) {
  f32x16 U = {}, V = {};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) U = Ty::mma32(fu(ks), Pu[ks], U);
#pragma unroll
  for (int s = 0; s < KS / 4; ++s) V = mma32x64_f8(fv(s), Pv[s], V);
  u32x4 Z[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      Z[s][q] = Ty::pack2(f8_gate<Ty>(U[8 * s + 2 * q], V[8 * s + 2 * q], deq),
                          f8_gate<Ty>(U[8 * s + 2 * q + 1], V[8 * s + 2 * q + 1], deq));
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int s = 0; s < 2; ++s) W[mb] = Ty::mma32(Z[s], fo(mb, s), W[mb]);
}

// Output of one 32-channel block of a pair: dl (lane = channel, register i = token kord(i)) is
// rounded to Ty; with RESIDUAL, x (the lane's token-side operands xk[0], xk[1], same tokens in
// the same order) is added and the sum rounded again, the reference's two rounding points
// (omniweave/models/block.py:87-108).  dst(i) is the element address of register i.  With
// SCALE, the rounded delta of token group 0 (registers 0..7) is multiplied by s0, that of group
// 1 by s1, and rounded again before the residual: the per-sample drop-path of training
// (block.py:99-107), where the scale is keep_mask * (1 / keep_probability) of the group's
// image and the reference's delta * keep_mask / keep_probability rounds once per product.
template <class Ty, bool RESIDUAL, bool SCALE = false, class Dst>
__device__ __forceinline__ void pair_store_block(const f32x16& dl, const u32x4 (&xk)[2], Dst dst, float s0 = 1.0f,
                                                 float s1 = 1.0f) {
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    uint32_t v = Ty::pack2(dl[i], dl[i + 1]);
    if constexpr (SCALE) {
      const float s = i < 8 ? s0 : s1;
      v = Ty::pack2(Ty::to_f32(lo16(v)) * s, Ty::to_f32(hi16(v)) * s);
    }
    if constexpr (RESIDUAL) {
      const uint32_t xp = xk[i >> 3][(i & 7) >> 1];
      v = Ty::pack2(Ty::to_f32(lo16(xp)) + Ty::to_f32(lo16(v)), Ty::to_f32(hi16(xp)) + Ty::to_f32(hi16(v)));
    }
    *dst(i) = lo16(v);
    *dst(i + 1) = hi16(v);
  }
}

// Output of one 32-channel block of a pair from delta^T (pair_output_t: lane l32 = token row,
// registers 4 q .. 4 q + 3 = channels 8 q + 4 hh .. + 3 of the block), in place in an LDS row
// tile that holds x: rounded to Ty (with SCALE times the drop-path scale s of the lane's token
// and rounded again, as pair_store_block), with RESIDUAL plus x read from the same positions,
// written back as 8-byte pieces.  at(q) is the LDS element pointer of the lane's run q.
template <class Ty, bool RESIDUAL, bool SCALE = false, class At>
__device__ __forceinline__ void pair_store_block_t(const f32x16& dl, At at, float s = 1.0f) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v0 = Ty::pack2(dl[4 * q], dl[4 * q + 1]);
    uint32_t v1 = Ty::pack2(dl[4 * q + 2], dl[4 * q + 3]);
    if constexpr (SCALE) {
      v0 = Ty::pack2(Ty::to_f32(lo16(v0)) * s, Ty::to_f32(hi16(v0)) * s);
      v1 = Ty::pack2(Ty::to_f32(lo16(v1)) * s, Ty::to_f32(hi16(v1)) * s);
    }
    u32x2* p = reinterpret_cast<u32x2*>(at(q));
    if constexpr (RESIDUAL) {
      const u32x2 x = *p;
      v0 = add_residual2<Ty>(x[0], v0);
      v1 = add_residual2<Ty>(x[1], v1);
    }
    *p = u32x2{v0, v1};
  }
}

// delta[mb] = A_o W[mb] for the pair; ao is the lane's A_o operand row (K step of its group).
template <class Ty, int MB>
__device__ __forceinline__ void pair_output(const f32x16 (&W)[MB], u32x4 ao, int lane, f32x16 (&dl)[MB]) {
  const bool g0 = (lane & 16) == 0;
  const u32x4 ao0 = keep_if(g0, ao), ao1 = keep_if(!g0, ao);
  const f32x16 zero = {};
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    dl[mb] = Ty::mma32(ao0, pack_kstep<Ty>(W[mb], 0), zero);
    dl[mb] = Ty::mma32(ao1, pack_kstep<Ty>(W[mb], 1), dl[mb]);
  }
}

// delta^T[mb] = W[mb]^T A_o^T for the pair (the same products as pair_output with the operands
// swapped): lane l32 = token l32 of the pair, register i = channel 32 mb + kord(i, hh), so a
// lane holds four runs of four consecutive channels of its token's row.
template <class Ty, int MB>
__device__ __forceinline__ void pair_output_t(const f32x16 (&W)[MB], u32x4 ao, int lane, f32x16 (&dl)[MB]) {
  const bool g0 = (lane & 16) == 0;
  const u32x4 ao0 = keep_if(g0, ao), ao1 = keep_if(!g0, ao);
  const f32x16 zero = {};
  // Both K steps of each block, the blocks interleaved so that no product waits on the one
  // issued right before it.
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) dl[mb] = Ty::mma32(pack_kstep<Ty>(W[mb], 0), ao0, zero);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) dl[mb] = Ty::mma32(pack_kstep<Ty>(W[mb], 1), ao1, dl[mb]);
}

inline int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return OW_OK;
  return fail(OW_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (cached per device id).
inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Persistent forward for d = 64, rd = 128 and C = q_c * 64 with q_c in {1, 2, 4}: weights of a
// channel group stay in the registers of one wave, one workgroup of q_c waves handles all
// channel groups of 32 tokens at a time (bigemm_fwd_resident.hip).
struct ResidentArgs {
  const uint16_t* x;
  uint16_t* out;
  const uint16_t* packed;  // packed weights, LayerScale folded (same layout as the streamed kernel)
  const int32_t* tok;      // [q_s * 16]
  const int32_t* chan;     // [q_c * 64]
  const int32_t* out_tok;  // [q_s * 16] output row of each token slot; NULL: the token table
  int32_t batch, n_tok, channels, q_s, q_c;
  int32_t n_pairs;  // ceil(batch * q_s / 2)
  int32_t norm;     // fuse the RMSNorm prologue
  int32_t residual; // write x + delta instead of delta
  float eps;
  const float* drop_scale;  // [batch] per-image multiplier of the rounded delta; NULL: none
  float* rs_out;            // 16-token kernel: the RMSNorm scale of every input row it normalises; NULL: none
};

bool resident_supported(int32_t d, int32_t rd, int32_t channels, int32_t q_c);

// Dispatch of a forward launch (bigemm_fwd.hip): the resident kernel (given rd = 2 d), or the
// streamed kernel's channel-group access mode; and whether the launch needs the batch * H * W
// fp32 RMSNorm row-scale buffer (statistics from a separate pass).
constexpr int kModeContig = 0;
constexpr int kModeStrided = 1;
constexpr int kModeElement = 2;
struct FwdPath {
  bool resident;
  int32_t mode;
};
FwdPath fwd_path(const void* x, const void* out, const OwPlan* plan, int32_t q_c, int32_t dtype, int32_t flags);
bool fwd_needs_scale_buffer(const void* x, const void* out, const OwPlan* plan, int32_t rd, int32_t dtype,
                            int32_t flags, bool stats_in, int32_t batch);
int launch_fwd_resident(const ResidentArgs& a, int32_t dtype, hipStream_t stream);
// Where the RMSNorm row scales of a streamed launch come from (bigemm_fwd.hip, FwdArgs).
constexpr int kNormNone = 0;
constexpr int kNormBuffer = 1;
constexpr int kNormInline = 2;
constexpr int kNormPartials = 3;


// Persistent d = 128 forward (bigemm_fwd_persist.hip): one eight-wave workgroup per CU over
// units of 256 rows x one contiguous channel group, the next unit's tile copied into LDS during
// the current unit's output phase.  RMSNorm scales from a statistics buffer or the previous
// block's per-group sums (norm: kNormNone, kNormBuffer or kNormPartials), or for strided groups
// from the whole rows the tile fetch reads (kNormInline).
struct PersistArgs {
  const uint16_t* x;
  uint16_t* out;
  const uint16_t* packed;
  const int32_t* tok;       // [q_s * 16]
  const int32_t* out_tok;   // [q_s * 16] output row of each token slot; NULL: the token table
  const float* row_scale;   // kNormBuffer: [batch * n_tok] scales; kNormPartials: [batch * n_tok, parts] sums
  float* stats_out;         // NULL, or [batch * n_tok, q_c]: sum of squares of each stored row's group columns
  const float* drop_scale;  // NULL, or [batch]: per-image multiplier of the rounded delta
  int32_t batch, n_tok, channels, q_s, q_c;
  int32_t norm;
  int32_t parts;
  float eps;
  int32_t residual;
  int32_t fp8;              // V' on the e4m3 MFMA (fp8 packed weights)
  const int32_t* chan;      // [q_c * 128] channel table (strided groups: the first entry of a group)
  int32_t stride;           // 1: contiguous groups; 2, 4, 8: strided groups (= q_c)
};
bool persist_supported(int32_t d, int32_t rd, int32_t channels, int32_t q_c, int64_t x_elems);
int launch_fwd_persist(const PersistArgs& a, int32_t dtype, hipStream_t stream);
// Whether a bf16 / f16 launch takes the persistent kernel.
bool fwd_uses_persist(const void* x, const void* out, const OwPlan* plan, int32_t rd, int32_t dtype, int32_t flags,
                      int32_t batch);

// 16-token-unit forward for d = 64, rd = 128, C = 64 q_c with q_c in {2, 4} (contiguous groups,
// or the interleaved groups of radix levels >= 1; bigemm_fwd_wave16.hip); reads the packed
// weights' second section (packed16_elems).
bool wave16_supported(int32_t d, int32_t rd, int32_t channels, int32_t q_c, int64_t x_elems);
int launch_fwd_wave16(const ResidentArgs& a, int32_t radix_level, int32_t dtype, hipStream_t stream);

// fp32 path (bigemm_fwd_f32.hip): operand packing, RMSNorm row scales and the forward.
int pack_weights_f32(const void* a_u, const void* a_v, const void* a_o, const void* b_u, const void* b_v,
                     const void* b_o, int32_t weight_dtype, const float* norm_weight, const float* gamma,
                     const int32_t* channel_index, int32_t channels, int32_t q_c, int32_t d, int32_t rd,
                     int64_t total, void* packed, hipStream_t stream);
int rms_scale_f32(const float* x, float* scale, int64_t rows, int32_t channels, float eps, hipStream_t stream);
int launch_fwd_f32(const float* x, float* out, const float* row_scale, const float* packed, const int32_t* tok,
                   const int32_t* chan, int32_t batch, int32_t n_tok, int32_t channels, int32_t q_s, int32_t q_c,
                   int32_t d, int32_t rd, int32_t residual, const float* drop_scale, hipStream_t stream);

// fp32 backward building blocks (bigemm_bwd_f32.hip).
int bwd_gather_f32(const float* x, const float* dy, const float* rscale, const int32_t* tok, const int32_t* chan,
                   float* xt, float* dyt, int64_t slots, int32_t n_tok, int32_t channels, int32_t q_s, int32_t q_c,
                   int32_t d, hipStream_t s);
int bwd_gate_f32(const float* u, const float* v, const float* dz, float* z, float* du, float* dv, int64_t n,
                 hipStream_t s);
int bwd_scatter_f32(const float* dxt, const int32_t* tok, const int32_t* chan, float* g, int64_t slots,
                    int32_t n_tok, int32_t channels, int32_t q_s, int32_t q_c, int32_t d, hipStream_t s);
int bwd_rmsnorm_f32(const float* x, const float* g, const float* rscale, const float* dout, float* dx, int64_t rows,
                    int32_t channels, int32_t residual, hipStream_t s);
int fold_weights_f32(const void* b_u, const void* b_v, const void* b_o, int32_t wdtype, const float* norm_w,
                     const float* gamma, const int32_t* chan, int32_t channels, int32_t q_c, int32_t d, int32_t rd,
                     float* bu, float* buT, float* bv, float* bvT, float* bo, float* boT, hipStream_t s);
int tile_mix_f32(const float* in1, const float* m1, const float* in2, const float* m2, float* out, int64_t n_tiles,
                 int32_t d, hipStream_t s);
int tile_outer_f32(const float* in1, const float* in2, float* partial, int32_t n_waves, int64_t n_tiles, int32_t d,
                   hipStream_t s);

}  // namespace ow
