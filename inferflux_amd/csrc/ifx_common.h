// ifx_common.h -- GGUF block formats and wave64 helpers shared by the gfx950
// kernels of the quantized GEMV/GEMM path.
//
// Block layouts follow the reference's structs
// (runtime/backends/cuda/native/kernels/dequantization.cuh:17-49,117-138):
//   Q4_K 144 B : u16 d | u16 dmin | u8 scales[12] | u8 qs[128]
//   Q6_K 210 B : u8 ql[128] | u8 qh[64] | i8 scales[16] | u16 d   (d last)
//   Q8_0  34 B : u16 d | i8 qs[32]
//   Q8_1  36 B : u16 d | u16 s (= d * sum(qs)) | i8 qs[32]
// The kernels address blocks as raw bytes (no packed structs), so rows whose
// byte stride is not a multiple of 16 (Q6_K, Q8_0) are read with plain
// loads at their natural offsets; gfx950 serves unaligned dword loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <initializer_list>

// Largest batch of the fused gate/up/SiLU kernel on wide Q4_K slices (one
// workgroup per batch column).  Measured at 11008 x 2048: from M = 3 on it
// loses to grouped GEMV + SiLU producer (M = 3 / 4 / 8: 12.6 / 14.5 / 23.0 us
// against 10.6 / 11.5 / 11.5 us): every column re-reads the weights.
#ifndef IFX_SWIGLU_MAX_M
#define IFX_SWIGLU_MAX_M 2
#endif

namespace ifx {

// Tuning overrides of the dispatch and launch geometry (IFX_PREFILL,
// IFX_DQ, IFX_SLOT_KW, ...) are read only in tuning builds (-DIFX_TUNING):
// a product build always takes the measured defaults the tests pin.
// Wave timelines for tuning builds (-DIFX_STAMPS): IFX_STAMP(k) has the
// lowest active lane of each wave of a launch write the constant 100 MHz clock to slot k (0..7)
// of its record in ifx_stamps (one record of 8 int64 per wave: region
// kStampBase (a constant the kernel defines, 0..3) of 16384 waves, then
// blockIdx.x major, then blockIdx.y, then the wave); the host reads the
// buffer through ifx_debug_stamps.  Product builds compile the macro to nothing.
#ifdef IFX_STAMPS
constexpr int kStampWaves = 1 << 16;
// one array per translation unit (no relocatable device code): a tuning
// build instruments the kernels of one file at a time (gemv.hip)
static __device__ long long ifx_stamps[kStampWaves * 8];
#define IFX_STAMP(k)                                                                              \
  do {                                                                                            \
    const long long t_ = static_cast<long long>(__builtin_amdgcn_s_memrealtime());                \
    const int w_ = kStampBase * 16384 +                                                           \
                   (static_cast<int>(blockIdx.x) * static_cast<int>(gridDim.y) +                  \
                    static_cast<int>(blockIdx.y)) * static_cast<int>(blockDim.x >> 6) +           \
                   static_cast<int>(threadIdx.x >> 6);                                            \
    const unsigned long long b_ = __ballot(1);                                                    \
    if (static_cast<unsigned long long>(threadIdx.x & 63) ==                                      \
            static_cast<unsigned long long>(__ffsll(static_cast<long long>(b_)) - 1) &&            \
        w_ < kStampWaves)                                                                         \
      ifx_stamps[w_ * 8 + (k)] = t_;                                                              \
  } while (0)
#else
#define IFX_STAMP(k) \
  do {               \
  } while (0)
#endif

inline const char *tuning_env(const char *name) {
#ifdef IFX_TUNING
  return getenv(name);
#else
  (void)name;
  return nullptr;
#endif
}

// Launch log: every kernel launch goes through IFX_LAUNCH, which records the
// instance name ("k_gemv<12,1,2,1,4,0,2>": the kernel's template arguments as
// integers) while a log is open on the calling thread, and skips the launch
// itself in dry-run mode (ifx_launch_log_begin, include/ifx_qgemm.h), so the
// dispatch can be inspected on a host without a GPU.
bool note_launch(const char *kernel, std::initializer_list<int> targs);
bool dry_run();
// hipGetLastError / hipPeekAtLastError, or hipSuccess in dry-run mode.
hipError_t last_error();
hipError_t peek_error();

#define IFX_UNPAREN(...) __VA_ARGS__
#define IFX_LAUNCH(K, TARGS, ...)                                        \
  do {                                                                   \
    if (::ifx::note_launch(#K, {IFX_UNPAREN TARGS}))                     \
      hipLaunchKernelGGL((K<IFX_UNPAREN TARGS>), __VA_ARGS__);           \
  } while (0)
#define IFX_LAUNCH0(K, ...)                                              \
  do {                                                                   \
    if (::ifx::note_launch(#K, {})) hipLaunchKernelGGL(K, __VA_ARGS__);  \
  } while (0)

constexpr int kTypeQ8_0 = 8;
constexpr int kTypeQ8_1 = 9;
constexpr int kTypeQ4_K = 12;
constexpr int kTypeQ5_K = 13;
constexpr int kTypeQ6_K = 14;
constexpr int kTypeQ8_K = 15;

constexpr int kQ4KBytes = 144;
constexpr int kQ5KBytes = 176;  // u16 d, u16 dmin, scales[12], qh[32], qs[128]
constexpr int kQ8KBytes = 292;  // f32 d, i8 qs[256], i16 bsums[16]
constexpr int kQ6KBytes = 210;
constexpr int kQ8_0Bytes = 34;
constexpr int kQ8_1Bytes = 36;

// Row-split layouts of this library (ifx_repack): each row's fields in
// separate 16-byte-aligned sections instead of interleaved GGUF blocks, so
// the M <= 2 GEMV reads them with aligned, fully used 16-byte loads.
//   Q8_0_R  [qs: K bytes][d: K/32 fp16][pad to 16]
//   Q6_K_R  [ql: K/2][qh: K/4][scales: K/16][d: K/256 fp16][pad to 16]
// The values are the GGUF block's bytes, moved.
constexpr int kTypeQ8_0R = 108;
constexpr int kTypeQ6_KR = 114;

// Tiled layouts of this library (ifx_repack_tiled): the rows in groups of
// 32, and per group and super-block one tile that holds the group's 32
// super-blocks with their bytes in the order the batch kernels' lanes load
// them (lane l: row l % 32, 16-byte pieces of K half l / 32), so each wave
// load instruction reads one contiguous kilobyte.  Tiles are ordered group
// major; the rows of a last, partial group are zero.
//   Q4_K_T (4608 B): [0, 512)   the 16-byte header (d, dmin, scales) of row c at 16 c
//                    512 + 1024 p + 512 h + 16 c: qs bytes 32 p + 16 h .. +15 of row c
//   Q6_K_T (6720 B): 1024 i + 512 h + 16 c: ql bytes 32 i + 16 h .. +15 (i = 0..3)
//                    4096 + 1024 g + 512 h + 16 c: qh bytes 32 g + 16 h .. +15 (g = 0, 1)
//                    6144 + 16 c: scales[16];  6656 + 2 c: d
//   Q8_0_T (8704 B, per 256 values): 1024 j + 512 h + 16 c: codes 16 h .. +15
//                    of block j (j = 0..7);  8192 + 16 c + 2 j: d of block j
constexpr int kTypeQ8_0T = 208;
constexpr int kTypeQ4_KT = 212;
constexpr int kTypeQ6_KT = 214;
constexpr int kTileRows = 32;

// Bytes of one weight row of K values.
__host__ __device__ constexpr int row_bytes(int qt, int K) {
  return (qt == kTypeQ4_K || qt == kTypeQ4_KT) ? (K >> 8) * kQ4KBytes
         : qt == kTypeQ6_KT ? (K >> 8) * kQ6KBytes
         : qt == kTypeQ5_K  ? (K >> 8) * kQ5KBytes
         : qt == kTypeQ6_K  ? (K >> 8) * kQ6KBytes
         : qt == kTypeQ8_K  ? (K >> 8) * kQ8KBytes
         : qt == kTypeQ8_0R ? ((K + (K >> 5) * 2 + 15) & ~15)
         : qt == kTypeQ6_KR ? (((K >> 1) + (K >> 2) + (K >> 4) + (K >> 8) * 2 + 15) & ~15)
                            : (K >> 5) * kQ8_0Bytes;
}

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// A constant in a VGPR, opaque to constant folding.  gfx950's VOP3
// encodings take no literal, so a mask-and-insert against a literal
// (x & mask) | magic compiles to v_and + v_or; with the magic in a register
// it is one v_and_or_b32 (the mask goes to an SGPR).
__device__ __forceinline__ uint32_t vreg(uint32_t c) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  _Float16 h;
  uint16_t b = static_cast<uint16_t>(bits16);
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32 default mode).
__device__ __forceinline__ uint32_t f2h_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Forces x to be rounded to an fp32 register value.  Without it the
// compiler may fuse "fp32 multiply, then convert to fp16" into a single
// mixed-precision FMA (one rounding instead of two), which changes results
// that must match an fp32-then-fp16 evaluation bit for bit.
__device__ __forceinline__ float materialize_f32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <typename T>
__device__ __forceinline__ T ldg(const void *p) {
  T v;
  __builtin_memcpy(&v, p, sizeof(T));
  return v;
}

// Buffer resources: a 32-bit byte range over a tensor.  Loads take a
// per-lane offset and a wave-uniform offset (scalar register), so address
// arithmetic stays 32-bit, and reads past the range return zeros.  Word 3 is
// the gfx9-family default (raw buffer, 32-bit dword format).
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// An offset past every W and A range the entry points accept (they refuse
// tensors of kMaxBufferBytes or more): a load there reads zeros and touches
// no memory.  Kernels add at most one weight tile or one Q8_1 row (K <=
// 2^24: 18.9 MB) to it, which stays below 2^32 whether or not the range
// check counts the scalar offset.
constexpr uint32_t kOobOffset = 0xF0000000u;
constexpr uint64_t kMaxBufferBytes = kOobOffset;

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, static_cast<int>(bytes),
                                           0x00020000);
}

template <typename T>
__device__ __forceinline__ T bload(rsrc_t r, uint32_t voff, uint32_t soff) {
  if constexpr (sizeof(T) == 16)
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  else if constexpr (sizeof(T) == 8)
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  else if constexpr (sizeof(T) == 4)
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
  else
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
}

// Cache policy of the weight-stream loads (buffer instruction aux bits).
#ifndef IFX_WAUX
#define IFX_WAUX 0
#endif
template <typename T>
__device__ __forceinline__ T wload(rsrc_t r, uint32_t voff, uint32_t soff) {
  if constexpr (sizeof(T) == 16)
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, IFX_WAUX));
  else if constexpr (sizeof(T) == 8)
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, IFX_WAUX));
  else if constexpr (sizeof(T) == 4)
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, IFX_WAUX));
  else
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, IFX_WAUX));
}

// DPP lane moves (VALU, no LDS): `old` is kept where the row/bank mask
// disables the move.
template <int CTRL, int ROWS = 0xF, int BANKS = 0xF>
__device__ __forceinline__ uint32_t dpp(uint32_t old, uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      static_cast<int>(old), static_cast<int>(v), CTRL, ROWS, BANKS, false));
}
template <int CTRL, int ROWS = 0xF, int BANKS = 0xF>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(float, dpp<CTRL, ROWS, BANKS>(0u, __builtin_bit_cast(uint32_t, v)));
}

// Sum over the 64 lanes of a wave with DPP adds; the total is exact in lane
// 63 (other lanes hold partial sums): quad swaps, half-row and row mirrors,
// then row 15 -> rows 1 and 3, lane 31 -> rows 2 and 3.
__device__ __forceinline__ float wave_sum_to63(float v) {
  v += dppf<0xB1>(v);         // quad_perm [1,0,3,2]
  v += dppf<0x4E>(v);         // quad_perm [2,3,0,1]
  v += dppf<0x141>(v);        // row_half_mirror
  v += dppf<0x140>(v);        // row_mirror
  v += dppf<0x142, 0xA>(v);   // row_bcast:15 into rows 1, 3
  v += dppf<0x143, 0xC>(v);   // row_bcast:31 into rows 2, 3
  return v;
}

// Sums over lanes 0-31 and over lanes 32-63 (two independent halves): the
// first five steps of wave_sum_to63; lane 31 and lane 63 hold the totals.
__device__ __forceinline__ float halfwave_sum_to31(float v) {
  v += dppf<0xB1>(v);
  v += dppf<0x4E>(v);
  v += dppf<0x141>(v);
  v += dppf<0x140>(v);
  v += dppf<0x142, 0xA>(v);
  return v;
}

// Sums over each 16-lane row (four independent quarters): the first four
// steps of wave_sum_to63; every lane of a row ends with its row's total.
__device__ __forceinline__ float quarterwave_sum(float v) {
  v += dppf<0xB1>(v);
  v += dppf<0x4E>(v);
  v += dppf<0x141>(v);
  v += dppf<0x140>(v);
  return v;
}

// Lane 8k's value in lanes 8k .. 8k+7 (row_newbcast of lanes 0 and 8 of
// each 16-lane row into banks 0-1 and 2-3).
__device__ __forceinline__ uint32_t bcast8(uint32_t v) {
  uint32_t x = dpp<0x150, 0xF, 0x3>(0u, v);
  return dpp<0x158, 0xF, 0xC>(x, v);
}

// Signed int8x4 dot product with int32 accumulate: v_dot4_i32_i8.
__device__ __forceinline__ int dot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Waits until every memory operation this wave issued has completed (its
// device-coherent stores included).  The compiler fences keep the memory
// operations around it on their side.
__device__ __forceinline__ void wait_own_memory() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Device-coherent fp32 store / load (relaxed, agent scope): data that other
// workgroups of the same launch read, on any XCD, without cache write-back
// or invalidation.
__device__ __forceinline__ void st_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Ordered K-split reduction (the workspace entry points): every workgroup of
// a split tile stores its fp32 partial sums to its own workspace slot with
// st_dev, each wave waits for its stores (wait_own_memory), and the
// workgroup then counts itself in on the tile's counter.  The workgroup that
// arrives last adds the slots in split order 0, 1, ... (ld_dev), so the
// result does not depend on which workgroup finishes last, applies the
// epilogue and resets the counter to zero for the next launch.  No
// workgroup waits for another, so no co-residency is assumed.  Returns true
// in the last workgroup (all threads).
struct SplitWs {
  uint32_t *cnt;  // one counter per tile, zero between launches
  float *part;    // partial-sum slots
};
__device__ __forceinline__ bool split_arrive_last(uint32_t *cnt, int ks) {
  __shared__ uint32_t last;
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           static_cast<uint32_t>(ks - 1);
  __syncthreads();
  return last != 0;
}
__device__ __forceinline__ void split_reset(uint32_t *cnt) {
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Zeroes up to three fp32 outputs before a split-K launch adds into them
// (mmq_skinny.hip); blockIdx.y selects the output.
struct FillArgs {
  float *y[3];
  int64_t n[3];
};
__global__ void k_fill_zero(const FillArgs f);
// Zeroes the first nseg outputs of f (one launch).  Returns the launch
// status without clearing it (hipPeekAtLastError).
hipError_t launch_fill_zero(const FillArgs &f, int nseg, hipStream_t s);

}  // namespace ifx
