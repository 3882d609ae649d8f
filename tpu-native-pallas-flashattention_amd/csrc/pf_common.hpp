// Shared device-side definitions for the gfx950 attention kernels.
//
// Element types: float (F32), __bf16 (BF16), _Float16 (F16). Every kernel
// upcasts to float32 and accumulates in float32 (the reference's arithmetic,
// flash_attention.py:91-93), feeding the MFMA matrix cores with the storage
// type (bf16/f16 operands, or float32 operands for F32 inputs).
//
// MFMA lane layouts used throughout (verified on gfx950 with an in-bounds
// probe: every output element of a random integer product matched):
//   v_mfma_f32_32x32x16_{bf16,f16}: A[32 x 16]: lane l holds A[l%32][8(l/32)+t],
//     t = 0..7; B[16 x 32]: lane l holds B[8(l/32)+t][l%32];
//     C[32 x 32]: lane l, register r holds C[8(r/4) + 4(l/32) + r%4][l%32].
//   v_mfma_f32_32x32x2f32: A: lane l holds A[l%32][l/32]; B: B[l/32][l%32];
//     C as above.
// A reduction (k) index can be assigned to (step, lane half, slot) in any
// bijective way as long as both operands agree; the kernels use that freedom
// so each lane half owns a contiguous range of the reduction dimension.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace pf {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;
typedef bf16_t bf16x8 __attribute__((ext_vector_type(8)));
typedef f16_t f16x8 __attribute__((ext_vector_type(8)));
typedef bf16_t bf16x4 __attribute__((ext_vector_type(4)));
typedef f16_t f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

// dtype tags shared with the C ABI (pf_dtype).
enum : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int kPerChunk = 4;  // elements per 16-byte chunk
  __device__ static inline float to_f32(float x) { return x; }
  __device__ static inline float from_f32(float x) { return x; }
};
template <>
struct Elem<bf16_t> {
  static constexpr int kPerChunk = 8;
  __device__ static inline float to_f32(bf16_t x) { return (float)x; }
  __device__ static inline bf16_t from_f32(float x) { return (bf16_t)x; }
};
template <>
struct Elem<f16_t> {
  static constexpr int kPerChunk = 8;
  __device__ static inline float to_f32(f16_t x) { return (float)x; }
  __device__ static inline f16_t from_f32(float x) { return (f16_t)x; }
};

// 32x32 MFMA with float32 accumulation. kK = reduction elements one lane
// supplies per instruction; Frag = that operand fragment.
template <typename T>
struct Mfma32;

template <>
struct Mfma32<bf16_t> {
  static constexpr int kK = 8;
  typedef bf16x8 Frag;
  __device__ static inline f32x16 run(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma32<f16_t> {
  static constexpr int kK = 8;
  typedef f16x8 Frag;
  __device__ static inline f32x16 run(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma32<float> {
  static constexpr int kK = 1;
  typedef float Frag;
  __device__ static inline f32x16 run(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// Number of MFMA operand fragments held in one 16-byte chunk.
template <typename T>
constexpr int frags_per_chunk() {
  return 16 / (Mfma32<T>::kK * (int)sizeof(T));
}

// Bits [lo, hi) of a 32-bit word, lo and hi clamped to [0, 32] (0 when the
// range is empty): the valid values of a lane's 32 scores in one step.
__device__ inline uint32_t bit_range(int lo, int hi) {
  lo = lo < 0 ? 0 : lo;
  hi = hi > 32 ? 32 : hi;
  if (hi <= lo) return 0u;
  const uint32_t top = hi >= 32 ? 0xffffffffu : (1u << hi) - 1u;
  return top & ~((1u << lo) - 1u);
}

// Bit i of m sign-extended over a word (all ones or zero): v_bfe_i32,
// written as assembly because the compiler rewrites a one-bit sign extension
// into AND + compare + select. i must be a constant once the caller's loops
// are unrolled (0..31). An ordinary VALU operation on a VGPR that integer
// VALU code computes (bit_range): none of the hazards the compiler would pad
// around it (MFMA results, transcendental results, SGPR writes) can reach
// its operand, so the statement needs no wait states of its own.
__device__ inline uint32_t bit_sel(uint32_t m, int i) {
  uint32_t sel;
  asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(sel) : "v"(m), "i"(i));
  return sel;
}

// v where bit i of m is set, +0.0 where it is clear: two VALU operations
// (extract, AND), no compare or branch, and a masked value that overflowed to
// inf still becomes exactly 0.
__device__ inline float keep_if_bit(float v, uint32_t m, int i) {
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & bit_sel(m, i));
}

// Workgroups per CU the 256-thread prefill and decode kernels are built for
// (the second __launch_bounds__ argument): 1 where a wave needs more than
// 256 registers (float32 at head_dim 128, every type at head_dim 256) or a
// workgroup more than half the LDS, else 2.
template <typename T, int D>
inline constexpr int kWgPerCu = ((sizeof(T) == 4 && D == 128) || D > 128) ? 1 : 2;

// Reinterpret a 16-byte chunk as operand fragment i.
template <typename T>
__device__ inline typename Mfma32<T>::Frag chunk_frag(const u32x4& c, int i) {
  if constexpr (sizeof(T) == 4) {
    // Cast the whole vector, then index: this compiler mis-lowers
    // __builtin_bit_cast(float, c[i]) on an ext-vector element (it reads
    // element 0 for every i).
    return __builtin_bit_cast(f32x4, c)[i];
  } else {
    return __builtin_bit_cast(typename Mfma32<T>::Frag, c);
  }
}

// Unpack a 16-byte chunk into float32 values (kPerChunk of them).
template <typename T>
__device__ inline void chunk_to_f32(const u32x4& c, float* out) {
  if constexpr (sizeof(T) == 4) {
    const f32x4 x = __builtin_bit_cast(f32x4, c);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = x[i];
  } else {
    typedef T v8 __attribute__((ext_vector_type(8)));
    v8 x = __builtin_bit_cast(v8, c);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = Elem<T>::to_f32(x[i]);
  }
}

// Pack kPerChunk float32 values into a 16-byte chunk of T (round to nearest even).
template <typename T>
__device__ inline u32x4 f32_to_chunk(const float* in) {
  if constexpr (sizeof(T) == 4) {
    const f32x4 x = {in[0], in[1], in[2], in[3]};
    return __builtin_bit_cast(u32x4, x);
  } else {
    typedef T v8 __attribute__((ext_vector_type(8)));
    v8 x;
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = Elem<T>::from_f32(in[i]);
    return __builtin_bit_cast(u32x4, x);
  }
}

// Wave-uniform raw buffer descriptor over [base, base + bytes), for the
// inline-assembly LDS DMA below (base and bytes must be wave-uniform). Loads
// at byte offsets at or past `bytes` return zeros without touching memory
// (hardware bounds check): that is how rows past kv_len, past a page's valid
// rows or past Sq are zero-filled without branches.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
__device__ inline i32x4 make_desc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 d;
  d[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  d[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  d[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  d[3] = 0x00020000;
  return d;
}

// Direct global -> LDS load of 64 lanes x 16 bytes (buffer_load_dwordx4 ...
// lds): lane l's chunk at byte `voff` of the buffer lands at LDS byte
// lds_addr + 16 l (lds_addr wave-uniform); lanes at or past the descriptor's
// size write zeros.
// Issued from inline assembly on purpose: the compiler treats an LDS DMA it
// can see as a possible alias of every later LDS read and makes the wave wait
// for all outstanding DMA (vmcnt(0)) before the first such read, which
// serialises a double-buffered pipeline on the global-load latency. The
// kernels instead wait explicitly (wait_vm) before the barrier that publishes
// a DMA'd buffer. The compiler's hazard recognizer cannot see inside inline
// assembly, so the asm pads the two gfx9-family hazards in front of an LDS
// DMA itself: the descriptor SGPRs come from v_readfirstlane (a VALU write of
// an SGPR read by a VMEM instruction needs 5 wait states) and the LDS address
// travels in M0 (an SALU write of M0 read by an LDS DMA needs 1). s_nop 4
// gives 5.
// NT = true marks the load non-temporal (the nt cache-policy bit): for data
// read once, such as a decode step's K/V stream, which should not displace
// reused lines from the caches.
template <bool NT = false>
__device__ inline void dma16(const i32x4& desc, uint32_t voff, uint32_t lds_addr) {
  // readfirstlane pins the (uniform) descriptor to SGPRs at this point, where
  // register pressure could otherwise leave it in VGPRs.
  i32x4 sd;
#pragma unroll
  for (int i = 0; i < 4; ++i) sd[i] = __builtin_amdgcn_readfirstlane(desc[i]);
  if constexpr (NT)
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "{m0}"(lds_addr), "v"(voff), "s"(sd)
                 : "memory");
  else
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "{m0}"(lds_addr), "v"(voff), "s"(sd)
                 : "memory");
}

// A burst of LDS DMA loads from one descriptor: dma_pin moves the descriptor
// into SGPRs once (readfirstlane) and pads the VALU-writes-SGPR hazard there,
// once, in an asm statement that takes the four values as tied operands, so
// every use comes after the pad; dma16_pinned then pads only the M0 write
// (1 wait state) in front of each load. The prefill kernels issue several
// loads per descriptor, each of which dma16 pads with 5 wait states.
__device__ inline i32x4 dma_pin(const i32x4& desc) {
  int a = __builtin_amdgcn_readfirstlane(desc[0]);
  int b = __builtin_amdgcn_readfirstlane(desc[1]);
  int c = __builtin_amdgcn_readfirstlane(desc[2]);
  int d = __builtin_amdgcn_readfirstlane(desc[3]);
  asm volatile("s_nop 4" : "+s"(a), "+s"(b), "+s"(c), "+s"(d));
  return (i32x4){a, b, c, d};
}
template <bool NT = false>
__device__ inline void dma16_pinned(const i32x4& sd, uint32_t voff, uint32_t lds_addr) {
  if constexpr (NT)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "{m0}"(lds_addr), "v"(voff), "s"(sd)
                 : "memory");
  else
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "{m0}"(lds_addr), "v"(voff), "s"(sd)
                 : "memory");
}

// Wait until at most N vector-memory loads of this wave are outstanding
// (loads complete in issue order).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

__device__ inline uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ inline u32x4 ldg16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ inline void stg16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
// Non-temporal forms, for streams touched once (copies into a cache or page
// pool, a rotation pass): they reach a higher HBM rate than ordinary loads
// and stores and leave the caches to data that is reused.
__device__ inline u32x4 ldg16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ inline void stg16_nt(void* p, u32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p)); }
__device__ inline u32x4 lds16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ inline void sts16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Reductions over the lane pair (l, l ^ 32) with v_permlane32_swap (a VALU
// swap of the wave's upper half of one register with the lower half of
// another): swapping x with itself yields x[l] and x[l ^ 32] in every lane,
// with no LDS round trip. Both results are symmetric in the pair, and
// a + b == b + a exactly, so both lane halves get bit-identical values.
__device__ inline f32x2 lane_pair(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return (f32x2){__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ inline float wave_xor32_max(float x) {
  const f32x2 v = lane_pair(x);
  return fmaxf(v[0], v[1]);
}
__device__ inline float wave_xor32_sum(float x) {
  const f32x2 v = lane_pair(x);
  return v[0] + v[1];
}

// f(std::integral_constant<int, i>{}) for i = 0 .. N-1, each call inlined with
// i a compile-time constant (a fully unrolled loop whose index can select
// registers and `if constexpr` branches).
template <typename F, int... I>
__device__ __attribute__((always_inline)) inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __attribute__((always_inline)) inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
// The same over i = LO .. HI-1 (empty when HI <= LO).
template <int LO, typename F, int... I>
__device__ __attribute__((always_inline)) inline void static_for_from(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, LO + I>{}), ...);
}
template <int LO, int HI, typename F>
__device__ __attribute__((always_inline)) inline void static_for_range(F&& f) {
  if constexpr (HI > LO) static_for_from<LO>(f, std::make_integer_sequence<int, HI - LO>{});
}

// Workgroup -> work-item remap that keeps the `group` consecutive work items
// (the query heads of one GQA group) on one XCD. Workgroups are dispatched
// round-robin over the 8 XCDs (XCD = blockIdx % 8); each XCD has its own L2,
// so items sharing K/V tiles should share an XCD. Bijective on [0, n).
__device__ inline int xcd_remap(int bid, int n, int group) {
  const int span = 8 * group;
  const int full = (n / span) * span;
  if (bid >= full) return bid;
  const int xcd = bid & 7;
  const int slot = bid >> 3;
  const int chunk = (slot / group) * 8 + xcd;
  return chunk * group + (slot % group);
}

}  // namespace pf
