// kcommon.hpp -- types and device helpers shared by the gfx950 kernels.
//
// Lane layouts of the MFMA instructions used here (wave64, lane l):
//   v_mfma_f32_32x32x2_f32   A: A[m = l%32][k = l/32]      B: B[k = l/32][n = l%32]
//   v_mfma_f32_32x32x16_bf16 A: A[m = l%32][k = 8(l/32)+j] B: B[k = 8(l/32)+j][n = l%32], j = 0..7
//   (f16 the same)
//   32x32 accumulator (16 regs): D[m = 8(i/4) + 4(l/32) + i%4][n = l%32], i = 0..15
//   v_mfma_f32_16x16x32_bf16 A: A[m = l%16][k = 8(l/16)+j] B: B[k = 8(l/16)+j][n = l%16], j = 0..7
//   16x16 accumulator (4 regs):   D[m = 4(l/16) + i][n = l%16], i = 0..3
// Any permutation of k applied identically to A and B leaves the product
// unchanged; the attention kernels use that to feed softmax probabilities to
// the second MFMA straight from the first MFMA's accumulator registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lchip::k {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Storage tags for the two 16-bit MFMA input formats.
struct BF16 {};
struct F16 {};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// fp32 -> fp16 bits, round to nearest even (hardware conversion).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

template <typename T>
__device__ __forceinline__ uint16_t to_half_bits(float f);
template <>
__device__ __forceinline__ uint16_t to_half_bits<BF16>(float f) {
  return f32_to_bf16_bits(f);
}
template <>
__device__ __forceinline__ uint16_t to_half_bits<F16>(float f) {
  return f32_to_f16_bits(f);
}

// Two fp32 values -> one packed dword of 16-bit values (lo in bits 0..15).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(to_half_bits<T>(lo)) | (static_cast<uint32_t>(to_half_bits<T>(hi)) << 16);
}
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}
// One v_cvt_pk_f16_f32 (round to nearest even, as the scalar conversion)
// instead of two conversions and an OR.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  f16x2 v;
  v[0] = static_cast<_Float16>(lo);
  v[1] = static_cast<_Float16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

// acc + lo + hi of a packed 16-bit pair, in one fp32 dot-product
// instruction (v_dot2c_f32_{bf16,f16} against (1, 1)).
template <typename T>
__device__ __forceinline__ float add_pair(uint32_t pair, float acc);
template <>
__device__ __forceinline__ float add_pair<BF16>(uint32_t pair, float acc) {
  const bf16x2 ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), ones, acc, false);
}
template <>
__device__ __forceinline__ float add_pair<F16>(uint32_t pair, float acc) {
  const f16x2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), ones, acc, false);
}

// max over lanes l and l ^ 32 (v_permlane32_swap: no LDS round trip).
__device__ __forceinline__ float max_xor32(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, r[0]), __builtin_bit_cast(float, r[1]));
}

// 32x32x16 MFMA on 8 packed 16-bit values per lane (as four dwords).
template <typename T>
__device__ __forceinline__ floatx16 mfma32x32x16(u32x4 a, u32x4 b, floatx16 c);
template <>
__device__ __forceinline__ floatx16 mfma32x32x16<BF16>(u32x4 a, u32x4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
template <>
__device__ __forceinline__ floatx16 mfma32x32x16<F16>(u32x4 a, u32x4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// 16x16x32 MFMA on 8 packed 16-bit values per lane (as four dwords).
template <typename T>
__device__ __forceinline__ floatx4 mfma16x16x32(u32x4 a, u32x4 b, floatx4 c);
template <>
__device__ __forceinline__ floatx4 mfma16x16x32<BF16>(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
template <>
__device__ __forceinline__ floatx4 mfma16x16x32<F16>(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

__device__ __forceinline__ floatx16 mfma32x32x2f32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 zero16() {
  floatx16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    z[i] = 0.0f;
  }
  return z;
}

// 16-byte global -> LDS copy of one lane from a wave-uniform base and a
// 32-bit per-lane byte offset (LDS address = lds + 16*lane), written as
// inline asm for two reasons:
//  * the scalar-base form needs no per-lane 64-bit address: a tile's lane
//    offsets are fixed, so a load costs one M0 move, and the wave issues the
//    copy instead of a stream of 64-bit address adds (measured on the 8192^3
//    bf16 GEMM: 1150 -> 1240 TFLOP/s);
//  * the compiler's wait-count pass does not see it.  An outstanding
//    compiler-visible global -> LDS copy makes every later LDS wait an
//    lgkmcnt(0), which stalls each MFMA group on LDS reads issued for the
//    next one.  Callers wait for these copies with explicit vmcnt.
// `lds` and `sbase` must be wave-uniform.  The LDS address reaches M0 through
// an "{m0}" input operand, so the compiler itself writes M0 (and knows its
// value afterwards); the asm never writes M0.
// Hazards: the compiler pads its own instructions for hardware hazards but not
// the contents of an asm statement.  A VALU write of an SGPR (v_readlane /
// v_readfirstlane, e.g. when the compiler reloads a spilled SGPR into the base
// pair) needs 5 wait states before a VMEM instruction reads that SGPR; with
// fewer the load can take a stale half of the 64-bit base and fault.  So the
// asm first copies the base with an SALU move (SALU reads of VALU-written
// SGPRs are interlocked) and the load reads the copy; that move is also the
// one wait state an SALU write of M0 needs before an LDS-DMA load reads M0.
// (tests/test_asm_hazards.py scans the built kernels for both.)
__device__ __forceinline__ void load_lds16_sbase(uint32_t voff, const void* sbase, uint32_t lds) {
  uint64_t base;
  asm volatile("s_mov_b64 %0, %2\n\tglobal_load_lds_dwordx4 %1, %0"
               : "=&s"(base)
               : "v"(voff), "s"(sbase), "{m0}"(lds)
               : "memory");
}

// The same copy with an instruction offset OFF (0..4095 bytes), which the
// hardware adds to both the global and the LDS address (measured on gfx950:
// lane l's 16 bytes from sbase + voff + OFF land at lds + OFF + 16*l).  Copies
// that fill consecutive 1 KB blocks of LDS can then share one M0 value, with
// OFF = 1024 * j and voff reduced by the same OFF.
template <int OFF>
__device__ __forceinline__ void load_lds16_sbase_off(uint32_t voff, const void* sbase, uint32_t lds) {
  static_assert(OFF >= 0 && OFF < 4096, "instruction offset");
  uint64_t base;
  asm volatile("s_mov_b64 %0, %2\n\tglobal_load_lds_dwordx4 %1, %0 offset:%3"
               : "=&s"(base)
               : "v"(voff), "s"(sbase), "i"(OFF), "{m0}"(lds)
               : "memory");
}

// The first of several copies that share one base (and one M0 value): the
// asm copies the base pair with an SALU move, as load_lds16_sbase_off does,
// issues the copy at instruction offset 0 and returns the pair it copied, so
// the copies after it (load_lds16_pair_off) read an SGPR pair whose last
// writer is that SALU move.  One move per part instead of one per copy
// (measured on the 8192^3 bf16 GEMM: 12 fewer SALU instructions per stage,
// 1531 -> 1562 TFLOP/s).  The hazard scan in tests/test_asm_hazards.py checks
// the built code for VALU writes of the pair within 5 wait states of a copy.
__device__ __forceinline__ uint64_t load_lds16_sbase_first(uint32_t voff, const void* sbase, uint32_t lds) {
  uint64_t pair;
  asm volatile("s_mov_b64 %0, %2\n\tglobal_load_lds_dwordx4 %1, %0"
               : "=&s"(pair)
               : "v"(voff), "s"(sbase), "{m0}"(lds)
               : "memory");
  return pair;
}

// A later copy of the same base pair and M0 value at instruction offset OFF
// (M0 must not change between the first copy and this one: the compiler
// keeps it, since every copy names the same value as its "{m0}" input).
template <int OFF>
__device__ __forceinline__ void load_lds16_pair_off(uint32_t voff, uint64_t pair, uint32_t lds) {
  static_assert(OFF > 0 && OFF < 4096, "instruction offset");
  asm volatile("global_load_lds_dwordx4 %0, %1 offset:%2" : : "v"(voff), "s"(pair), "i"(OFF), "{m0}"(lds) : "memory");
}

// LDS byte address of a __shared__ object, as a wave-uniform value.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}

// s_waitcnt vmcnt(n) (expcnt / lgkmcnt left at their maxima; vmcnt's low
// four bits sit in bits 3:0 of the immediate, its high two in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(n) (vmcnt / expcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt immediate");
  __builtin_amdgcn_s_waitcnt((0xc07f & ~(0xf << 8)) | (N << 8));
}

// Workgroup barrier without the release fence of __syncthreads(): the fence
// would make the compiler drain every outstanding global -> LDS load
// (vmcnt(0)) at each stage and collapse a multi-stage pipeline.  Callers wait
// for exactly the stage they need with s_waitcnt vmcnt(n) first; every LDS
// read of the retiring stage has already been consumed by its MFMA.  The empty
// asm statements keep the compiler from moving memory operations across.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Row (m) index held by accumulator register i of lane l in a 32x32 tile.
__device__ __forceinline__ int acc_row(int i, int lane) {
  return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}

// Optional completion flag of a synchronous small call: `flag` is a
// host-mapped word the host spins on, `count` a device counter that starts at
// zero.  Each workgroup makes its output visible to the host (system-scope
// release) before thread 0 counts it with an acquire-release add at device
// scope, so the last workgroup's count follows every other workgroup's
// release; the last one zeroes the counter for the next launch and publishes
// `seq` with a system-scope release store.
struct DoneFlag {
  unsigned* count = nullptr;
  unsigned* flag = nullptr;
  unsigned seq = 0;
  // With a flag, the attention kernels let wave 0 store the workgroup's whole
  // output, so one wave's release covers it.
  __device__ bool single_writer() const { return flag != nullptr; }
  // Every thread, after wave 0 stored the workgroup's whole output.
  __device__ void finish() const {
    if (flag == nullptr || threadIdx.x >= 64) {
      return;
    }
    __threadfence_system();
    if (threadIdx.x == 0) {
      count_and_publish();
    }
  }
  // Every thread, after storing its own share of the output: each wave
  // releases its stores, then the barrier orders them before the count.
  __device__ void finish_all_writers() const {
    if (flag == nullptr) {
      return;
    }
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
      count_and_publish();
    }
  }
  __device__ void count_and_publish() const {
    const unsigned total = gridDim.x * gridDim.y * gridDim.z;
    if (__hip_atomic_fetch_add(count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == total - 1) {
      __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __threadfence_system();
      __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
};

}  // namespace lchip::k
