// fwl_common.h -- shared by the HIP sources of libfwloss.so: buffer-resource access, element
// types, wavefront primitives (DPP, permlane swaps, ballots), the candidate-list solve and small
// host helpers.  Everything is in an anonymous namespace, so each source file has its own copy.
#pragma once
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wunused-function"
#pragma clang diagnostic ignored "-Wunneeded-internal-declaration"
#pragma clang diagnostic ignored "-Wunused-const-variable"

// Compile with -Xclang -target-feature -Xclang -packed-fp32-ops (see fwloss_build.py).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <atomic>
#include <map>
#include <type_traits>
#include <mutex>
#include <utility>

#include "fwloss.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer resources (GFX9 layout): the hardware range check drops stores and zero-fills loads
// past `bytes`, so every lane can issue the same unconditional instruction.  Memory instructions
// under lane-dependent branches would make the compiler's wait counting fall back to draining all
// outstanding stores at the top of each row.
constexpr int kRsrcFlags = 0x00020000;
constexpr int kNonTemporal = 2;   // cache-policy bits of the buffer instructions: nt
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kRsrcFlags);
}

// Element types of the logits (and of the gradient of the fused op): float, or the 16-bit tags
// below.  Values are widened to fp32 exactly when loaded; every decision is taken in fp32/fp64;
// gradient values are computed in fp32 and rounded to nearest-even when stored.
struct bf16_t {};   // bfloat16, stored as uint16
struct f16_t {};    // IEEE binary16, stored as uint16
template <typename T> constexpr int kElemBytes = 2;
template <> constexpr int kElemBytes<float> = 4;
template <typename T> using Storage = typename std::conditional<std::is_same<T, float>::value, float, uint16_t>::type;

// elements per lane access: a 128-bit unit (VEC) or a single element
template <typename T, bool VEC> constexpr int kUnit = VEC ? 16 / kElemBytes<T> : 1;

template <typename T>
__device__ __forceinline__ float widen16(uint32_t h) {
  if constexpr (std::is_same<T, bf16_t>::value) return __uint_as_float(h << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <typename T>
__device__ __forceinline__ uint32_t narrow16(float f) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;   // NaN stays NaN (quiet)
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;                     // round to nearest even
  } else {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  }
}

// unit `u` of a row (elements kUnit*u ...) as fp32; offsets past the resource read 0
template <typename T, bool VEC>
__device__ __forceinline__ void load_unit(rsrc_t r, uint32_t u, float* out) {
  if constexpr (VEC) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, 16u * u, 0, kNonTemporal);
    if constexpr (std::is_same<T, float>::value) {
      out[0] = __uint_as_float(v.x);
      out[1] = __uint_as_float(v.y);
      out[2] = __uint_as_float(v.z);
      out[3] = __uint_as_float(v.w);
    } else {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[2 * i] = widen16<T>(w[i] & 0xFFFFu);
        out[2 * i + 1] = widen16<T>(w[i] >> 16);
      }
    }
  } else if constexpr (std::is_same<T, float>::value) {
    out[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, 4u * u, 0, kNonTemporal));
  } else {
    out[0] = widen16<T>(__builtin_amdgcn_raw_buffer_load_b16(r, 2u * u, 0, kNonTemporal));
  }
}

// store unit `u` (kUnit values, rounded to T); offsets past the resource are dropped
template <typename T, bool VEC>
__device__ __forceinline__ void store_unit(rsrc_t r, uint32_t u, const float* v) {
  if constexpr (VEC) {
    v4u w;
    if constexpr (std::is_same<T, float>::value) {
      w = v4u{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
    } else {
      w = v4u{narrow16<T>(v[0]) | (narrow16<T>(v[1]) << 16), narrow16<T>(v[2]) | (narrow16<T>(v[3]) << 16),
              narrow16<T>(v[4]) | (narrow16<T>(v[5]) << 16), narrow16<T>(v[6]) | (narrow16<T>(v[7]) << 16)};
    }
    __builtin_amdgcn_raw_buffer_store_b128(w, r, 16u * u, 0, kNonTemporal);
  } else if constexpr (std::is_same<T, float>::value) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, 4u * u, 0, kNonTemporal);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)narrow16<T>(v[0]), r, 2u * u, 0, kNonTemporal);
  }
}

// bit pattern of an fp32 value in element type T (16-bit types: in the low half)
template <typename T>
__device__ __forceinline__ uint32_t encode(float f) {
  if constexpr (std::is_same<T, float>::value) return __float_as_uint(f);
  else return narrow16<T>(f);
}

// store unit `u` from already-encoded element bit patterns
// (POL: cache policy; the non-temporal hint suits streams that read and write, a pure write
// stream runs faster without it)
template <typename T, bool VEC, int POL = kNonTemporal>
__device__ __forceinline__ void store_unit_bits(rsrc_t r, uint32_t u, const uint32_t* b) {
  if constexpr (VEC) {
    v4u w;
    if constexpr (std::is_same<T, float>::value) w = v4u{b[0], b[1], b[2], b[3]};
    else w = v4u{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
    __builtin_amdgcn_raw_buffer_store_b128(w, r, 16u * u, 0, POL);
  } else if constexpr (std::is_same<T, float>::value) {
    __builtin_amdgcn_raw_buffer_store_b32(b[0], r, 4u * u, 0, POL);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)b[0], r, 2u * u, 0, POL);
  }
}

// a zero unit (all-zero bits are +0 in every element type)
template <typename T, bool VEC>
__device__ __forceinline__ void store_zero_unit(rsrc_t r, uint32_t u) {
  if constexpr (VEC) __builtin_amdgcn_raw_buffer_store_b128(v4u{0u, 0u, 0u, 0u}, r, 16u * u, 0, kNonTemporal);
  else if constexpr (std::is_same<T, float>::value) __builtin_amdgcn_raw_buffer_store_b32(0u, r, 4u * u, 0, kNonTemporal);
  else __builtin_amdgcn_raw_buffer_store_b16((uint16_t)0, r, 2u * u, 0, kNonTemporal);
}

// scalar element access through plain pointers (element index j)
template <typename T>
__device__ __forceinline__ float load_elem(const void* base, int64_t j) {
  if constexpr (std::is_same<T, float>::value) return static_cast<const float*>(base)[j];
  else return widen16<T>(static_cast<const uint16_t*>(base)[j]);
}
template <typename T>
__device__ __forceinline__ void store_elem(void* base, int64_t j, float v) {
  if constexpr (std::is_same<T, float>::value) static_cast<float*>(base)[j] = v;
  else static_cast<uint16_t*>(base)[j] = (uint16_t)narrow16<T>(v);
}

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;
constexpr int kMaxWaveC = 2048;        // longest row held in registers by one wavefront (128-bit rows)
constexpr int kMaxWaveC1 = 1024;       // the same for rows accessed 32 bits at a time
constexpr int kMaxStreamC = 8192;      // longest row streamed by one wavefront (longer: one block per row)
constexpr int kCapMax = 512;           // LDS candidate slots per wavefront in fwl_block_rows
constexpr int kMaxBlocksWave = 2048;   // grid cap of fwl_wave_rows (4 rows in flight per block)
constexpr int kMaxBlocksRow = 4096;    // grid cap of fwl_block_rows
constexpr int kStreamUnroll = 4;       // 128-bit loads per lane per streaming round
constexpr int kRoundSlotsV1 = 16;      // 32-bit loads per lane per streaming round (unaligned rows)
constexpr size_t kWsAlign = 256;       // alignment of the workspace's parts
constexpr uint32_t kOffNone = 0x7FFFFFF0u;   // a buffer offset past every resource: access dropped

enum Mode : int { kGrad = 0, kMask = 1, kCand = 2 };

struct Outs {
  float* H;
  float* loss;
  float* mean;         // the mean loss (null: none requested)
  double* loss64;      // optional fp64 per-row losses (the value `loss` rounds)
  int32_t* kappa;
  void* grad;   // element type of the logits
  uint8_t* mask;
  float* cval;
  int32_t* cidx;
  int32_t* ccnt;
  double scale;        // gradient scale (1/N for the mean reduction)
  double reduce_div;   // mean = sum(losses) / reduce_div
  float scale_f;
  double* partials;    // one fp64 loss sum per block (null: no mean requested)
  float* ovf_lo;       // streaming kernels: per row, a lower bound on tau for rows whose lists
  float* ovf_mx;       // overflowed (NaN for the others) and the row maximum; null: no deferral
  int64_t ld;          // row stride of the logits, in elements (>= C)
  int force_generic;
  int cap;             // LDS candidate capacity per wavefront (<= kCapMax)
  int cstride;         // candidate-list mode: row stride of cval/cidx (C for the drop-in op)
  int ccap;            // candidate-list mode: entries kept per row (further ones are dropped)
  int mark_unlisted;   // candidate-list mode: a row whose list kept values only gets ccnt = -kappa
                       // (support not listed) instead of one more pass over the row to list it
};

// ------------------------------------------------------------------------------------------------
// wavefront primitives (all lanes of the wavefront must be active when these are called)

__device__ __forceinline__ int lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// a 64-bit value the whole wavefront holds, in scalar registers (for row addresses that the
// compiler cannot prove uniform, e.g. ones derived from LDS loads: buffer instructions with a
// resource in vector registers are wrapped in loops over the distinct values)
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// make_rsrc for a base address and size that the whole wavefront shares, forced into scalar
// registers (the compiler may hold a row pointer derived from a spilled kernel argument in vector
// registers; a buffer instruction with such a resource runs in a loop over its distinct values)
__device__ __forceinline__ rsrc_t make_rsrc_u(const void* base, uint32_t bytes) {
  const int64_t b = uniform64(reinterpret_cast<int64_t>(base));
  return make_rsrc(reinterpret_cast<const void*>(b), (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes));
}

// number of set bits of b in lanes below this one
__device__ __forceinline__ int rank_in(uint64_t b) {
  return __builtin_amdgcn_mbcnt_hi((unsigned)(b >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)b, 0u));
}

// DPP controls (GFX9 encoding)
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kRowRor8 = 0x128;       // row_ror:8  (lane ^ 8 inside a row of 16)
constexpr int kRowMirror = 0x140;     // lane 15 - i inside a row of 16
constexpr int kRowHalfMirror = 0x141; // lane 7 - i inside a half row of 8
constexpr int kRowBcast15 = 0x142;    // lane 15 of each row to the next row
constexpr int kRowBcast31 = 0x143;    // lane 31 to rows 2 and 3

template <int CTRL>
__device__ __forceinline__ int dpp_mov(int x) {
  return __builtin_amdgcn_mov_dpp(x, CTRL, 0xF, 0xF, false);
}

// lanes whose DPP source is out of range (or whose row is masked off) read 0
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_or0(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROW_MASK, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ double dpp_mov_f64(double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = dpp_mov<CTRL>((int)b);
  const int hi = dpp_mov<CTRL>((int)(b >> 32));
  return __longlong_as_double((int64_t)(((uint64_t)(unsigned)hi << 32) | (unsigned)lo));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_or0_f64(double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = dpp_or0<CTRL, ROW_MASK>((int)b);
  const int hi = dpp_or0<CTRL, ROW_MASK>((int)(b >> 32));
  return __longlong_as_double((int64_t)(((uint64_t)(unsigned)hi << 32) | (unsigned)lo));
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const int64_t b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)b, l);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
  return __longlong_as_double((int64_t)(((uint64_t)(unsigned)hi << 32) | (unsigned)lo));
}

// partner value of lane ^ M, without LDS: DPP inside rows of 16 lanes, the gfx950 permlane swaps
// across rows (v_permlane16_swap / v_permlane32_swap with both operands x return, per lane, the
// value of the other row / half in r[1] for the lower and r[0] for the upper one)
template <int M>
__device__ __forceinline__ float xor_lane(float v, int lane) {
  const int x = __float_as_int(v);
  if constexpr (M == 1) return __int_as_float(dpp_mov<kQuadXor1>(x));
  else if constexpr (M == 2) return __int_as_float(dpp_mov<kQuadXor2>(x));
  else if constexpr (M == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, false);   // row_shl:4
    const int dn = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);   // row_shr:4
    return __int_as_float((lane & 4) ? dn : up);
  } else if constexpr (M == 8) return __int_as_float(dpp_mov<kRowRor8>(x));
  else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return __int_as_float((lane & 16) ? r[0] : r[1]);
  } else {
    static_assert(M == 32, "xor distance");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return __int_as_float((lane & 32) ? r[0] : r[1]);
  }
}

// per-lane select with a wavefront-constant lane mask held in SGPRs (one v_cndmask)
__device__ __forceinline__ float select_lanes(uint64_t mask, float if_set, float if_clear) {
  float r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(if_clear), "v"(if_set), "s"(mask));
  return r;
}

// maximum over the wavefront, returned in every lane (wavefront-uniform)
// fp32 sum over the wavefront in a fixed order (for bounds: each value takes part in at most 6
// roundings of the tree, see safe_lower32)
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += __int_as_float(dpp_mov<kQuadXor1>(__float_as_int(v)));
  v += __int_as_float(dpp_mov<kQuadXor2>(__float_as_int(v)));
  v += __int_as_float(dpp_mov<kRowHalfMirror>(__float_as_int(v)));
  v += __int_as_float(dpp_mov<kRowMirror>(__float_as_int(v)));
  const int x = __float_as_int(v);
  const float a = __int_as_float(__builtin_amdgcn_readlane(x, 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(x, 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(x, 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(x, 48));
  return (a + b) + (c + d);
}

__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, __int_as_float(dpp_mov<kQuadXor1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<kQuadXor2>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<kRowHalfMirror>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<kRowMirror>(__float_as_int(v))));
  const int x = __float_as_int(v);
  const float a = __int_as_float(__builtin_amdgcn_readlane(x, 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(x, 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(x, 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(x, 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// fp64 sum over the wavefront in a fixed order, returned in every lane
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_mov_f64<kQuadXor1>(v);
  v += dpp_mov_f64<kQuadXor2>(v);
  v += dpp_mov_f64<kRowHalfMirror>(v);
  v += dpp_mov_f64<kRowMirror>(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

// integer sum over the wavefront, returned in every lane
__device__ __forceinline__ int wave_sum_i32(int v) {
  v += dpp_mov<kQuadXor1>(v);
  v += dpp_mov<kQuadXor2>(v);
  v += dpp_mov<kRowHalfMirror>(v);
  v += dpp_mov<kRowMirror>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

__device__ __forceinline__ double wave_max_f64(double v) {
  v = fmax(v, dpp_mov_f64<kQuadXor1>(v));
  v = fmax(v, dpp_mov_f64<kQuadXor2>(v));
  v = fmax(v, dpp_mov_f64<kRowHalfMirror>(v));
  v = fmax(v, dpp_mov_f64<kRowMirror>(v));
  return fmax(fmax(readlane_f64(v, 0), readlane_f64(v, 16)), fmax(readlane_f64(v, 32), readlane_f64(v, 48)));
}

// one compare-exchange step of a bitonic network sorting groups of K lanes (descending where
// lane & K == 0); the lanes keeping the maximum form a constant mask
constexpr uint64_t keep_max_mask(int K, int J) {
  uint64_t m = 0;
  for (int i = 0; i < 64; ++i)
    if (((i & J) == 0) == ((i & K) == 0)) m |= 1ull << i;
  return m;
}

template <int K, int J>
__device__ __forceinline__ float bitonic_step(float v, int lane) {
  const float p = xor_lane<J>(v, lane);
  return select_lanes(keep_max_mask(K, J), fmaxf(v, p), fminf(v, p));
}

template <int K>
__device__ __forceinline__ float bitonic_merge(float v, int lane) {
  if constexpr (K >= 64) v = bitonic_step<K, 32>(v, lane);
  if constexpr (K >= 32) v = bitonic_step<K, 16>(v, lane);
  if constexpr (K >= 16) v = bitonic_step<K, 8>(v, lane);
  if constexpr (K >= 8) v = bitonic_step<K, 4>(v, lane);
  if constexpr (K >= 4) v = bitonic_step<K, 2>(v, lane);
  return bitonic_step<K, 1>(v, lane);
}

// Order-preserving integer key of a float that is not NaN: signed comparison of keys orders the
// values (-0.0 just below +0.0).  The map is its own inverse.  Integer max/min need no NaN
// quieting, so a compare-exchange is a DPP max, a DPP min and one select.
__device__ __forceinline__ int fkey(float v) {
  const int b = __float_as_int(v);
  return b ^ ((b >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float fkey_inv(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7FFFFFFF)); }

// partner of lane ^ M for integer values; lane ^ 4 takes two bank-masked DPP moves (banks 0 and 2
// of each row, lanes with bit 2 clear, read lane + 4 = row_ror:12; banks 1 and 3 read lane - 4 =
// row_ror:4)
template <int M>
__device__ __forceinline__ int xor_lane_i(int x, int lane) {
  if constexpr (M == 1) return dpp_mov<kQuadXor1>(x);
  else if constexpr (M == 2) return dpp_mov<kQuadXor2>(x);
  else if constexpr (M == 4) {
    const int a = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0x5, false);
    return __builtin_amdgcn_update_dpp(a, x, 0x124, 0xF, 0xA, false);
  } else if constexpr (M == 8) return dpp_mov<kRowRor8>(x);
  else return __float_as_int(xor_lane<M>(__int_as_float(x), lane));
}

__device__ __forceinline__ int select_lanes_i(uint64_t mask, int if_set, int if_clear) {
  int r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(if_clear), "v"(if_set), "s"(mask));
  return r;
}

template <int K, int J>
__device__ __forceinline__ int bitonic_step_i(int v, int lane) {
  const int p = xor_lane_i<J>(v, lane);
  return select_lanes_i(keep_max_mask(K, J), max(v, p), min(v, p));
}

template <int K>
__device__ __forceinline__ int bitonic_merge_i(int v, int lane) {
  if constexpr (K >= 64) v = bitonic_step_i<K, 32>(v, lane);
  if constexpr (K >= 32) v = bitonic_step_i<K, 16>(v, lane);
  if constexpr (K >= 16) v = bitonic_step_i<K, 8>(v, lane);
  if constexpr (K >= 8) v = bitonic_step_i<K, 4>(v, lane);
  if constexpr (K >= 4) v = bitonic_step_i<K, 2>(v, lane);
  return bitonic_step_i<K, 1>(v, lane);
}

// sort the keys of lanes [0, T) descending (T = 16, 32 or 64)
template <int T>
__device__ __forceinline__ int sort_desc_i(int v, int lane) {
  v = bitonic_merge_i<2>(v, lane);
  v = bitonic_merge_i<4>(v, lane);
  v = bitonic_merge_i<8>(v, lane);
  v = bitonic_merge_i<16>(v, lane);
  if constexpr (T >= 32) v = bitonic_merge_i<32>(v, lane);
  if constexpr (T >= 64) v = bitonic_merge_i<64>(v, lane);
  return v;
}

// DPP move whose lanes without a source (shifted in past the row edge) read 0
template <int CTRL>
__device__ __forceinline__ double dpp_zero_f64(double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_mov_dpp((int)b, CTRL, 0xF, 0xF, true);
  const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), CTRL, 0xF, 0xF, true);
  return __longlong_as_double((int64_t)(((uint64_t)(unsigned)hi << 32) | (unsigned)lo));
}

// inclusive prefix sum over lanes [0, T)
template <int T>
__device__ __forceinline__ double scan_f64(double v) {
  v += dpp_zero_f64<0x111>(v);          // row_shr:1
  v += dpp_zero_f64<0x112>(v);          // row_shr:2
  v += dpp_zero_f64<0x114>(v);          // row_shr:4
  v += dpp_zero_f64<0x118>(v);          // row_shr:8
  if constexpr (T >= 32) v += dpp_or0_f64<kRowBcast15, 0xA>(v);   // rows 1, 3 += last lane of 0, 2
  if constexpr (T >= 64) v += dpp_or0_f64<kRowBcast31, 0xC>(v);   // rows 2, 3 += lane 31
  return v;
}

// inclusive prefix sum of an int over the wavefront's 64 lanes
__device__ __forceinline__ int scan_i32(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0x111, 0xF, 0xF, true);   // row_shr:1 (past the row edge: 0)
  v += __builtin_amdgcn_mov_dpp(v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += __builtin_amdgcn_mov_dpp(v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += __builtin_amdgcn_mov_dpp(v, 0x118, 0xF, 0xF, true);   // row_shr:8
  v += dpp_or0<kRowBcast15, 0xA>(v);                          // rows 1, 3 += last lane of 0, 2
  v += dpp_or0<kRowBcast31, 0xC>(v);                          // rows 2, 3 += lane 31
  return v;
}

// largest float <= t (so that x > t <=> x > rd32(t) for every float x; fw_cpu.cpp:96-101)
__device__ __forceinline__ float rd32(double t) {
  float r = (float)t;
  if ((double)r > t) {
    unsigned b = __float_as_uint(r);
    if (r > 0.0f) b -= 1u;
    else if (r < 0.0f) b += 1u;
    else b = 0x80000001u;
    r = __uint_as_float(b);
  }
  return r;
}

// next float / double below a finite value
__device__ __forceinline__ float prev_f32(float r) {
  unsigned b = __float_as_uint(r);
  if (r > 0.0f) b -= 1u;
  else if (r < 0.0f) b += 1u;
  else b = 0x80000001u;
  return __uint_as_float(b);
}
__device__ __forceinline__ double prev_f64(double r) {
  uint64_t b = (uint64_t)__double_as_longlong(r);
  if (r > 0.0) b -= 1u;
  else if (r < 0.0) b += 1u;
  else b = 0x8000000000000001ull;
  return __longlong_as_double((int64_t)b);
}

// next float above a finite value
__device__ __forceinline__ float next_f32(float r) {
  unsigned b = __float_as_uint(r);
  if (r > 0.0f) b += 1u;
  else if (r < 0.0f) b -= 1u;
  else b = 1u;
  return __uint_as_float(b);
}

// A float strictly below H = (s - 1)/c, where s is the fp64 sum (any order) of c values of
// magnitude <= B: below the exact H of those values whatever the rounding of the sum (at most
// c*B*2^-53 per term added, so c*B*2^-53 after the division by c), of the subtraction and of the
// division.  H of any non-empty subset of a row is <= tau (fw_cpu.cpp:201-211), so the result is
// a safe lower bound on tau.  NaN/inf inputs give -inf (no bound).
__device__ __forceinline__ float safe_lower(double s, int c, float B) {
  if (c <= 0) return -INFINITY;
  const double h = (s - 1.0) / (double)c;
  const double err = ((double)c * (double)B + (fabs(s) + 1.0) / (double)c + fabs(h)) * 0x1p-51;
  const float r = rd32(h - err);
  return isfinite(r) ? prev_f32(r) : -INFINITY;
}

// safe_lower for a sum s accumulated partly in fp32: per-lane partial sums of at most 63 values of
// magnitude <= B each, then added in fp64.  Adding the j-th value rounds by at most j*B*2^-24, so
// a lane of k values is off by at most k(k+1)/2 * B*2^-24, and the error of the sum divided by the
// number c of values is at most (k_max + 1)/2 * B*2^-24 <= B*2^-19: the bound moves down by that.
// Lanes of at most 48 values may also be added by wave_sum_f32 instead: each of its 6 levels
// rounds by at most 2^-24 times the sum of the magnitudes below it (<= c*B), 6*B*2^-24 per value,
// and 24.5 + 6 < 32.
__device__ __forceinline__ float safe_lower32(double s, int c, float B) {
  if (c <= 0) return -INFINITY;
  const double h = (s - 1.0) / (double)c - (double)B * 0x1p-19;
  const double err = ((double)c * (double)B + (fabs(s) + 1.0) / (double)c + fabs(h)) * 0x1p-51;
  const float r = rd32(h - err);
  return isfinite(r) ? prev_f32(r) : -INFINITY;
}

// largest float <= m - 1 (tau >= m - 1, so every support entry is > this bound).  For |m| >= 2^53
// the fp64 subtraction loses the 1; the float below m is then the answer.
__device__ __forceinline__ float bound_below_max(float m) {
  const float t = rd32((double)m - 1.0);
  return (t >= m && isfinite(m)) ? prev_f32(m) : t;
}

// tau < max always; fp64 rounding can only violate this when the 1 of S - 1 is lost (|z| >= 2^53)
__device__ __forceinline__ double clamp_below_max(double tau, float m) {
  return (tau >= (double)m && isfinite(m)) ? prev_f64((double)m) : tau;
}

// tau of a candidate set held one value per lane in lanes [0, n), 1 <= n <= T <= 64: sort
// descending, S_k = fp64 prefix sums; tau = max_k (S_k - 1)/k (reference_impl.py:17-21).  The
// maximising k is the support size: k z_(k) > S_k - 1 holds exactly for k = 1 .. kappa (the
// sparsemax support condition; both sides are exact in fp64 whenever S_k is), so one division
// gives tau = (S_kappa - 1)/kappa.  Rounding is monotone, so this is the largest of the rounded
// (S_k - 1)/k.
template <int T>
__device__ __forceinline__ double select_tier(float c, int n, int lane) {
  int key = fkey(lane < n ? c + 0.0f : -INFINITY);   // + 0.0f: -0.0 -> +0.0
  key = sort_desc_i<T>(key, lane);
  const float v = fkey_inv(key);
  const double S = scan_f64<T>(lane < n ? (double)v : 0.0);
  const uint64_t in = ballot(lane < n && (double)v * (double)(lane + 1) > S - 1.0);
  int kap = 64 - (int)__builtin_clzll(in | 1ull);   // the highest k that satisfies it (>= 1)
  kap = uniform(kap);
  return (readlane_f64(S, kap - 1) - 1.0) / (double)kap;
}

__device__ __forceinline__ double select_small(float c, int n, int lane) {
  if (n <= 16) return select_tier<16>(c, n, lane);
  if (n <= 32) return select_tier<32>(c, n, lane);
  return select_tier<64>(c, n, lane);
}

// sum/count over the first n entries of one wavefront's list, entries > thr
__device__ __forceinline__ void list_sum_count(const float* bv, int n, float thr, int lane, double& s,
                                               int& c) {
  double acc = 0.0;
  int cnt = 0;
  for (int p0 = 0; p0 < n; p0 += kWave) {
    const int p = p0 + lane;
    const float v = p < n ? bv[p] : -INFINITY;
    const bool k = v > thr;
    acc += k ? (double)v : 0.0;
    cnt += __popcll(ballot(k));
  }
  s = wave_sum_f64(acc);
  c = cnt;
}

// Padded lists: storage of a whole number of 4*64-entry groups, 16-byte aligned.  pad_list sets
// the entries [n, n rounded up to 256) to -inf, after which a pass reads four entries per lane
// with one 128-bit LDS load and needs no bound check (-inf is above no threshold).
__device__ __forceinline__ void pad_list(float* bv, int n, int lane) {
  const int end = (n + 4 * kWave - 1) & ~(4 * kWave - 1);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q = n + lane + kWave * j;
    if (q < end) bv[q] = -INFINITY;
  }
}

// this lane's sum (in A: float for bounds, at most n/64 terms; double for exact steps) and count
// of the entries > thr of a padded list [0, n)
template <typename A>
__device__ __forceinline__ void list4_lane(const float* bv, int n, float thr, int lane, A& acc, int& cnt) {
  acc = (A)0;
  cnt = 0;
#pragma unroll 2
  for (int p0 = 0; p0 < n; p0 += 4 * kWave) {
    const v4f v = *reinterpret_cast<const v4f*>(bv + p0 + 4 * lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool k = v[j] > thr;
      acc += k ? (A)v[j] : (A)0;
      cnt += k ? 1 : 0;
    }
  }
}

// list_sum_count over a padded list, fp64
__device__ __forceinline__ void list4_sum_count(const float* bv, int n, float thr, int lane, double& s, int& c) {
  double acc;
  int cnt;
  list4_lane<double>(bv, n, thr, lane, acc, cnt);
  s = wave_sum_f64(acc);
  c = wave_sum_i32(cnt);
}

// list4_compact that also returns this lane's fp32 sum and count of the entries kept (at most n/64
// terms: a bound's partial sum, see safe_lower32)
__device__ __forceinline__ int list4_compact_sum(float* bv, int* bi, int n, float t, bool noidx, int lane,
                                                 float& ks, int& kc) {
  int w = 0;
  ks = 0.0f;
  kc = 0;
  for (int p0 = 0; p0 < n; p0 += 4 * kWave) {
    const int p = p0 + 4 * lane;
    const v4f v = *reinterpret_cast<const v4f*>(bv + p);
    v4i id = {-1, -1, -1, -1};
    if (!noidx) id = *reinterpret_cast<const v4i*>(bi + p);
    // every write below lands below p0 + 256: on entries this group has already read
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool keep = v[j] > t;
      ks += keep ? v[j] : 0.0f;
      kc += keep ? 1 : 0;
      const uint64_t b = ballot(keep);
      if (keep) {
        const int pos = w + rank_in(b);
        bv[pos] = v[j];
        if (!noidx) bi[pos] = id[j];
      }
      w += __popcll(b);
    }
    __builtin_amdgcn_wave_barrier();
  }
  return w;
}

// keep the entries > t of a padded list [0, n) in place (and their indices, unless noidx; bi is
// then padded storage too); returns the number kept.  The order of the entries changes.
__device__ __forceinline__ int list4_compact(float* bv, int* bi, int n, float t, bool noidx, int lane) {
  int w = 0;
  for (int p0 = 0; p0 < n; p0 += 4 * kWave) {
    const int p = p0 + 4 * lane;
    const v4f v = *reinterpret_cast<const v4f*>(bv + p);
    v4i id = {-1, -1, -1, -1};
    if (!noidx) id = *reinterpret_cast<const v4i*>(bi + p);
    // every write below lands below p0 + 256: on entries this group has already read
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool keep = v[j] > t;
      const uint64_t b = ballot(keep);
      if (keep) {
        const int pos = w + rank_in(b);
        bv[pos] = v[j];
        if (!noidx) bi[pos] = id[j];
      }
      w += __popcll(b);
    }
    __builtin_amdgcn_wave_barrier();
  }
  return w;
}

// tau, kappa and (for n <= 64) the support bits of a candidate list cl[0, n) that holds every row
// entry > t0 (t0 <= tau, e.g. the largest float <= max - 1) and whose largest entry is the row
// maximum m.  Up to 64 entries: one per lane, sorted across the wavefront, fp64 prefix sums,
// tau = max_k (S_k - 1)/k.  Longer lists: fixed-point iterations t <- H({z > t}) from t0 (each
// iterate is <= tau and the set shrinks every step until it is {z > tau}).
// (PAD: cl is a padded list, see pad_list, whose passes use 128-bit loads)
template <bool PAD = false>
__device__ __forceinline__ void resolve_list(const float* cl, int n, float t0, float m, int lane, double& tau,
                                             int& kappa, uint64_t& support) {
  auto sum_count = [&](float thr, double& s, int& c) {
    if constexpr (PAD) list4_sum_count(cl, n, thr, lane, s, c);
    else list_sum_count(cl, n, thr, lane, s, c);
  };
  tau = NAN;
  kappa = 0;
  support = 0;
  if (n > 0 && n <= kWave) {
    const float c = lane < n ? cl[lane] : -INFINITY;
    tau = clamp_below_max(select_small(c, n, lane), m);
    support = ballot(lane < n && c > rd32(tau));
    kappa = __popcll(support);
  } else if (n > kWave) {
    double t = (double)t0, s;
    int c;
    sum_count(t0, s, c);
    for (int it = 0; it <= n + 1; ++it) {
      const double tn = (s - 1.0) / (double)c;
      double s2;
      int c2;
      sum_count(rd32(tn), s2, c2);
      if (c2 == c || !(tn > t)) {
        tau = tn;
        kappa = c2;
        break;
      }
      t = tn;
      s = s2;
      c = c2;
    }
    const double tc = clamp_below_max(tau, m);
    if (tc != tau) {
      double s3;
      tau = tc;
      sum_count(rd32(tau), s3, kappa);
    }
  }
}

// ---- host helpers

inline int blocks_wave(int64_t N) {
  const int64_t b = (N + kWavesPerBlock - 1) / kWavesPerBlock;
  return (int)(b < kMaxBlocksWave ? (b > 0 ? b : 1) : kMaxBlocksWave);
}

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

inline int launch_status() { return hipGetLastError() == hipSuccess ? FWL_OK : FWL_ERR_LAUNCH; }

constexpr int64_t kMaxC = (int64_t)1 << 29;
inline bool bad_shape(int64_t N, int64_t C) { return N < 0 || C < 1 || C > kMaxC; }

}  // namespace

#pragma clang diagnostic pop
