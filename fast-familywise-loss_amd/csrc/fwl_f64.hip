// fwl_f64.hip -- float64 logits for libfwloss.so (fwl_forward_backward_f64, fwl_scale_grad_f64 of
// include/fwloss.h): the reference CPU path's second dtype (src/cpu/fw_cpu.cpp:697-703).
//
// Compile with -Xclang -target-feature -Xclang -packed-fp32-ops (see fwloss_build.py).
#include "fwl_common.h"

namespace {

// ------------------------------------------------------------------------------------------------
// fp64 logits (the reference CPU path's second dtype, src/cpu/fw_cpu.cpp:697-703): one wavefront per
// row.  The row is streamed once for its candidates z > (running max) - 1, kept in LDS; tau comes
// from fixed-point iterations t <- H({z > t}) on that list (Michelot), every sum in fp64 in a fixed
// order; a second stream of the row writes the gradient.  Rows whose candidates do not fit in the
// list run the same iterations over the whole row.

constexpr int kF64Cap = 1024;    // LDS candidates per wavefront (a round adds at most 512)
constexpr int kF64Round = 4;     // 128-bit units (two doubles) per lane per streaming round

// largest double <= m - 1 (the subtraction's rounding error from TwoSum)
__device__ __forceinline__ double bound_below_max_f64(double m) {
  const double s = m - 1.0;
  const double bp = s - m, ap = s - bp;
  const double e = (m - ap) + (-1.0 - bp);   // m - 1 == s + e exactly
  double t = e < 0.0 ? prev_f64(s) : s;
  if (t >= m && isfinite(m)) t = prev_f64(m);   // |m| >= 2^53: the 1 is lost
  return t;
}

__device__ __forceinline__ void sum_count_f64(const double* v, int n, double t, int lane, double& s, int& c) {
  double acc = 0.0;
  int cnt = 0;
  for (int p0 = 0; p0 < n; p0 += kWave) {
    const int p = p0 + lane;
    const double x = p < n ? v[p] : -INFINITY;
    const bool k = x > t;
    acc += k ? x : 0.0;
    cnt += __popcll(ballot(k));
  }
  s = wave_sum_f64(acc);
  c = cnt;
}

// two doubles of a 128-bit unit, one of a 64-bit unit
__device__ __forceinline__ double lo_f64(v4u w) { return __longlong_as_double((int64_t)(((uint64_t)w.y << 32) | w.x)); }
__device__ __forceinline__ double hi_f64(v4u w) { return __longlong_as_double((int64_t)(((uint64_t)w.w << 32) | w.z)); }
__device__ __forceinline__ double one_f64(v2u w) { return __longlong_as_double((int64_t)(((uint64_t)w.y << 32) | w.x)); }

// sum and count of the row entries > t (a stream of the row; EVEN: 128-bit units of two doubles)
template <bool EVEN>
__device__ __forceinline__ void row_sum_count_f64(rsrc_t row, int C, double t, int lane, double& s, int& c) {
  const int slots = EVEN ? C / 2 : C;
  double acc = 0.0;
  int cnt = 0;
  for (int u = lane; u - lane < slots; u += kWave) {
    double x0, x1 = -INFINITY;
    if constexpr (EVEN) {
      const v4u w = __builtin_amdgcn_raw_buffer_load_b128(row, 16u * (uint32_t)u, 0, kNonTemporal);
      x0 = u < slots ? lo_f64(w) : -INFINITY;
      x1 = u < slots ? hi_f64(w) : -INFINITY;
    } else {
      const v2u w = __builtin_amdgcn_raw_buffer_load_b64(row, 8u * (uint32_t)u, 0, kNonTemporal);
      x0 = u < slots ? one_f64(w) : -INFINITY;
    }
    acc += x0 > t ? x0 : 0.0;
    acc += x1 > t ? x1 : 0.0;
    cnt += (x0 > t) + (x1 > t);
  }
  s = wave_sum_f64(acc);
  c = (int)wave_sum_f64((double)cnt);
}

// Stable in-place compaction of an fp64 candidate list to its entries > t.
__device__ __forceinline__ int filter_f64(double* v, int n, double t, int lane) {
  int out = 0;
  for (int p0 = 0; p0 < n; p0 += kWave) {
    const int p = p0 + lane;
    const double x = p < n ? v[p] : -INFINITY;
    const bool keep = x > t;
    const uint64_t b = ballot(keep);
    __builtin_amdgcn_wave_barrier();
    if (keep) v[out + rank_in(b)] = x;
    out += __popcll(b);
    __builtin_amdgcn_wave_barrier();
  }
  return out;
}

// EVEN (C even): 128-bit accesses of two doubles; odd C: 64-bit accesses.
template <bool EVEN, int R>
__global__ __launch_bounds__(kBlock) void fwl_rows_f64(const double* __restrict__ z, const int64_t* __restrict__ tgt,
                                                       int64_t N, int C, double scale, double* __restrict__ H,
                                                       double* __restrict__ loss, int32_t* __restrict__ kappa,
                                                       double* __restrict__ grad) {
  __shared__ double s_val[kWavesPerBlock][kF64Cap];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  double* cl = s_val[wid];
  const uint32_t row_bytes = (uint32_t)(8 * C);
  for (int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid; r < N; r += stride) {
    const rsrc_t row = make_rsrc(z + r * C, row_bytes);
    // pass 1: candidates above the running bound
    double m = -INFINITY, t = -INFINITY;
    int n = 0;
    bool over = false;
    const int slots = EVEN ? C / 2 : C;   // 128-bit units, or single doubles
    // R > 0: the whole row in R rounds held in registers (no second read for the gradient)
    double xr[R > 0 ? R : 1][2 * kF64Round];
    auto round = [&](int u0, double* x) {
#pragma unroll
      for (int q = 0; q < kF64Round; ++q) {
        const int u = u0 + lane + kWave * q;
        if constexpr (EVEN) {
          const v4u w = __builtin_amdgcn_raw_buffer_load_b128(row, 16u * (uint32_t)u, 0, kNonTemporal);
          x[2 * q] = u < slots ? lo_f64(w) : -INFINITY;
          x[2 * q + 1] = u < slots ? hi_f64(w) : -INFINITY;
        } else {
          const v2u w = __builtin_amdgcn_raw_buffer_load_b64(row, 8u * (uint32_t)u, 0, kNonTemporal);
          x[2 * q] = u < slots ? one_f64(w) : -INFINITY;
          x[2 * q + 1] = -INFINITY;
        }
      }
      double lm = x[0];
#pragma unroll
      for (int i = 1; i < 2 * kF64Round; ++i) lm = fmax(lm, x[i]);
      const double wm = wave_max_f64(lm);
      if (wm > m) {
        m = wm;
        t = bound_below_max_f64(m);
      }
      if (!over) {
#pragma unroll
        for (int i = 0; i < 2 * kF64Round; ++i) {
          const bool c = x[i] > t;
          const uint64_t b = ballot(c);
          if (b != 0) {
            const int at = n + rank_in(b);
            if (c && at < kF64Cap) cl[at] = x[i];
            n += __popcll(b);
          }
        }
        __builtin_amdgcn_wave_barrier();
        // at most kF64Cap / 2 entries before a round, so nothing is dropped; more than that above
        // the current bound sends the row to the whole-row iterations
        if (n > kF64Cap / 2) n = filter_f64(cl, n, t, lane);
        if (n > kF64Cap / 2) over = true;
      }
    };
    if constexpr (R > 0) {
#pragma unroll
      for (int rd = 0; rd < R; ++rd) round(rd * kWave * kF64Round, xr[rd]);
    } else {
      for (int u0 = 0; u0 < slots; u0 += kWave * kF64Round) {
        double x[2 * kF64Round];
        round(u0, x);
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (!over) n = filter_f64(cl, n, t, lane);
    // tau by t <- H({z > t}) from t <= tau: each iterate is <= tau and the set shrinks until it is
    // the support (on the list, or on the whole row when the list overflowed)
    double tau = NAN;
    int kap = 0;
    if (over || n > 0) {
      double s;
      int c;
      if (over) row_sum_count_f64<EVEN>(row, C, t, lane, s, c);
      else sum_count_f64(cl, n, t, lane, s, c);
      for (int it = 0; it <= C + 1; ++it) {
        const double tn = (s - 1.0) / (double)c;
        double s2;
        int c2;
        if (over) row_sum_count_f64<EVEN>(row, C, tn, lane, s2, c2);
        else sum_count_f64(cl, n, tn, lane, s2, c2);
        if (c2 == c || !(tn > t) || c2 == 0) {
          tau = tn;
          kap = c2;
          break;
        }
        t = tn;
        s = s2;
        c = c2;
      }
      if (tau >= m && isfinite(m)) {   // tau < max always (fp64 loses the 1 only for |z| >= 2^53)
        tau = prev_f64(m);
        double s3;
        if (over) row_sum_count_f64<EVEN>(row, C, tau, lane, s3, kap);
        else sum_count_f64(cl, n, tau, lane, s3, kap);
      }
    }
    // outputs and pass 2: the gradient
    const int64_t y = tgt[r];
    const bool yok = y >= 0 && y < C;
    const double zy = yok ? z[r * C + y] : NAN;
    if (lane == 0) {
      if (H) H[r] = tau;
      if (loss) loss[r] = yok ? (1.0 - zy) + tau : NAN;
      if (kappa) kappa[r] = kap;
    }
    const double inv = scale / (double)kap;
    const rsrc_t out = make_rsrc(grad + r * C, row_bytes);
    if constexpr (R > 0) {
#pragma unroll
      for (int rd = 0; rd < R; ++rd) {
#pragma unroll
        for (int q = 0; q < kF64Round; ++q) {
          const int u = rd * kWave * kF64Round + lane + kWave * q;   // past the row: dropped
          const double x0 = xr[rd][2 * q], x1 = xr[rd][2 * q + 1];
          double g0 = x0 > tau ? inv : 0.0, g1 = x1 > tau ? inv : 0.0;
          if constexpr (EVEN) {
            if (yok && 2 * u == y) g0 -= scale;
            if (yok && 2 * u + 1 == y) g1 -= scale;
            const uint64_t b0 = (uint64_t)__double_as_longlong(g0), b1 = (uint64_t)__double_as_longlong(g1);
            __builtin_amdgcn_raw_buffer_store_b128(
                v4u{(uint32_t)b0, (uint32_t)(b0 >> 32), (uint32_t)b1, (uint32_t)(b1 >> 32)}, out, 16u * (uint32_t)u, 0,
                kNonTemporal);
          } else {
            if (yok && u == y) g0 -= scale;
            const uint64_t b0 = (uint64_t)__double_as_longlong(g0);
            __builtin_amdgcn_raw_buffer_store_b64(v2u{(uint32_t)b0, (uint32_t)(b0 >> 32)}, out, 8u * (uint32_t)u, 0,
                                                  kNonTemporal);
          }
        }
      }
      continue;
    }
    for (int u = lane; u - lane < slots; u += kWave) {
      if constexpr (EVEN) {
        const v4u w = __builtin_amdgcn_raw_buffer_load_b128(row, 16u * (uint32_t)u, 0, kNonTemporal);
        const double x0 = lo_f64(w), x1 = hi_f64(w);
        double g0 = x0 > tau ? inv : 0.0, g1 = x1 > tau ? inv : 0.0;
        if (yok && 2 * u == y) g0 -= scale;
        if (yok && 2 * u + 1 == y) g1 -= scale;
        const uint64_t b0 = (uint64_t)__double_as_longlong(g0), b1 = (uint64_t)__double_as_longlong(g1);
        __builtin_amdgcn_raw_buffer_store_b128(v4u{(uint32_t)b0, (uint32_t)(b0 >> 32), (uint32_t)b1, (uint32_t)(b1 >> 32)},
                                               out, 16u * (uint32_t)u, 0, kNonTemporal);
      } else {
        const v2u w = __builtin_amdgcn_raw_buffer_load_b64(row, 8u * (uint32_t)u, 0, kNonTemporal);
        const double x0 = one_f64(w);
        double g0 = x0 > tau ? inv : 0.0;
        if (yok && u == y) g0 -= scale;
        const uint64_t b0 = (uint64_t)__double_as_longlong(g0);
        __builtin_amdgcn_raw_buffer_store_b64(v2u{(uint32_t)b0, (uint32_t)(b0 >> 32)}, out, 8u * (uint32_t)u, 0,
                                              kNonTemporal);
      }
    }
  }
}

// mean = sum(losses) / reduce_div in a fixed order (one block)
__global__ __launch_bounds__(kBlock) void fwl_mean_f64(const double* __restrict__ loss, int64_t N, double reduce_div,
                                                       double* __restrict__ mean) {
  __shared__ double s_red[kBlock];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < N; i += kBlock) acc += loss[i];
  s_red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) s_red[threadIdx.x] += s_red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) *mean = s_red[0] / reduce_div;
}

// grad[r, :] *= grad_output[r * go_stride] (fp64) for rows whose factor is not 1
__global__ __launch_bounds__(kBlock) void fwl_scale_rows_f64(double* __restrict__ grad, const double* __restrict__ go,
                                                             int64_t go_stride, int64_t N, int C) {
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid; r < N; r += stride) {
    const double s = go[r * go_stride];
    if (s == 1.0) continue;
    for (int j = lane; j < C; j += kWave) grad[r * C + j] *= s;
  }
}

// ---- fp64 logits (host side)

int forward_f64(const double* z, const int64_t* y, int64_t N, int64_t C, double scale, double reduce_div, double* H,
                double* losses, double* mean, int32_t* kappa, double* grad, hipStream_t s) {
  if (bad_shape(N, C) || (N > 0 && (z == nullptr || y == nullptr || grad == nullptr)) ||
      (mean != nullptr && N > 0 && losses == nullptr))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(z, 8) || !aligned(y, 8) || !aligned(grad, 8) || !aligned(H, 8) || !aligned(losses, 8) ||
      !aligned(mean, 8) || !aligned(kappa, 4))
    return FWL_ERR_ALIGNMENT;
  if (N > 0) {
    // rows of up to 4 rounds stay in registers (512 doubles per round with 128-bit units, 256 with
    // 64-bit ones)
    const int per_round = (C % 2 == 0 ? 2 : 1) * kWave * kF64Round;
    const int rounds = (int)((C + per_round - 1) / per_round);
    const dim3 g(blocks_wave(N)), b(kBlock);
#define FWL_F64(E, R) hipLaunchKernelGGL((fwl_rows_f64<E, R>), g, b, 0, s, z, y, N, (int)C, scale, H, losses, kappa, grad)
    if (C % 2 == 0) {
      if (rounds <= 1) FWL_F64(true, 1);
      else if (rounds <= 2) FWL_F64(true, 2);
      else if (rounds <= 4) FWL_F64(true, 4);
      else FWL_F64(true, 0);
    } else {
      if (rounds <= 1) FWL_F64(false, 1);
      else if (rounds <= 2) FWL_F64(false, 2);
      else if (rounds <= 4) FWL_F64(false, 4);
      else FWL_F64(false, 0);
    }
#undef FWL_F64
  }
  if (mean != nullptr) hipLaunchKernelGGL(fwl_mean_f64, dim3(1), dim3(kBlock), 0, s, losses, N, reduce_div, mean);
  return launch_status();
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// C ABI

extern "C" {

int fwl_forward_backward_f64(const double* logits, const int64_t* targets, int64_t N, int64_t C, double scale,
                             double reduce_div, double* H, double* losses, double* mean_loss, int32_t* kappa,
                             double* grad, hipStream_t stream) {
  return forward_f64(logits, targets, N, C, scale, reduce_div, H, losses, mean_loss, kappa, grad, stream);
}

int fwl_scale_grad_f64(double* grad, const double* grad_output, int64_t go_stride, int64_t N, int64_t C,
                       hipStream_t stream) {
  if (bad_shape(N, C) || go_stride < 0 || (N > 0 && (grad == nullptr || grad_output == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(grad, 8) || !aligned(grad_output, 8)) return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  hipLaunchKernelGGL(fwl_scale_rows_f64, dim3(blocks_wave(N)), dim3(kBlock), 0, stream, grad, grad_output, go_stride, N,
                     (int)C);
  return launch_status();
}

}  // extern "C"
