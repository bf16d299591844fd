// libfwloss.so -- Familywise (FW) loss forward/backward for MI355X (gfx950), behind the C ABI of
// include/fwloss.h.
//
// Per row z (C fp32 logits) the threshold tau = max_k (S_k - 1)/k (reference_impl.py:11-35) is
// the root of sum_j max(z_j - tau, 0) = 1 (src/cpu/fw_cpu.cpp:1-4).  Two facts drive the design:
//   * tau >= max(z) - 1, so the support {z > tau} lies in (max - 1, max]: only a few entries per
//     row ("candidates") matter, the rest of the row is read once and written once;
//   * H(A) = (sum_A z - 1)/|A| <= tau for every non-empty subset A of the row, so any such value is
//     a lower bound that may be used to discard entries early (fw_cpu.cpp:201-211).
//
// Kernels
//   fwl_wave_rows   C <= 2048 (1024 for rows that are not 16-byte aligned): one wavefront per
//                   row, the row held in VGPRs (128-bit buffer loads),
//                   the next row's loads issued as soon as this row's candidates z > max-1 are
//                   compacted into an LDS list (prefix sum of per-lane counts, branch-free
//                   writes).  Up to 64 candidates are sorted across the wavefront (bitonic network
//                   over DPP and permlane swaps), prefix-summed in fp64 (DPP row_shr + row_bcast
//                   scan) and tau = max_k (S_k - 1)/k; longer lists use fixed-point (Michelot)
//                   iterations.  The epilogue writes the gradient / mask / candidate list; H, loss
//                   and kappa of a wavefront's rows are stored once after its last row.
//   fwl_wave_stream_rows  mid-range C (up to 8192): one wavefront per row, streamed as below with
//                   a single wavefront's list; no block-wide barrier.
//   fwl_block_rows  C > 8192: one block (4 wavefronts) per row.  Each wavefront streams its share
//                   of the row once, its loads one round ahead, with a running lower bound
//                   t = (its max so far) - 1; it keeps the entries z > t in an LDS list (value,
//                   index) and writes a zero placeholder for every output element as it goes.
//                   After the selection only the support entries and the label are rewritten,
//                   so almost every 128-byte line is written exactly once, whole.  A full list is
//                   tightened by fixed-point iterations on the list; a list that cannot be
//                   tightened sends the row to the generic multi-pass path.
//   fwl_mask_to_grad, fwl_cand_to_grad   the two-op backward of the drop-in interface.
// Other sources of the library: fwl_f64.hip (float64 logits), fwl_linear.hip (the LM head fused
// with the loss), fwl_common.h (what they share).
// The mean loss is reduced in fp64 in a fixed order: per-block partial sums, summed in a fixed
// lane-strided order by the last block to finish, found by one ticket (grids of up to 512 blocks) or by a ticket per
// group of 32 blocks whose last finishers share a second ticket (ticket counters in the caller's
// workspace, each reset by its last user).
//
#include "fwl_common.h"

namespace {

// ------------------------------------------------------------------------------------------------
// mean of the per-row losses: each block stores its fp64 partial sum; fwl_mean_finish, launched
// after the rows on the same stream, adds the partials in a fixed order.  No counters: the
// workspace holds no state from one call to the next.

// Wait until this thread's earlier vector memory operations have completed (stores acknowledged).
// Unlike a device-scope fence this does not write back the L2 cache.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Called by every thread of a block with the block's loss sum (thread 0's value is used).
__device__ __forceinline__ void mean_epilogue(double bsum, const Outs& o) {
  if (o.partials != nullptr && threadIdx.x == 0) o.partials[blockIdx.x] = bsum;
}

// One wavefront: lane l adds partials l, l + 64, l + 128, ... in turn (loads issued kSumBatch at a
// time, so that their round trips overlap), then a butterfly over the lanes (x + y == y + x, so
// every lane ends with the same bits); mean = total / reduce_div.
constexpr int kSumBatch = 8;
__global__ __launch_bounds__(kWave) void fwl_mean_finish(const double* __restrict__ p, unsigned nb,
                                                        double reduce_div, float* __restrict__ mean) {
  const unsigned lane = threadIdx.x;
  double acc = 0.0;
  for (unsigned base = 0; base < nb; base += kWave * kSumBatch) {
    double v[kSumBatch];
#pragma unroll
    for (int k = 0; k < kSumBatch; ++k) {
      const unsigned i = base + lane + kWave * k;
      v[k] = i < nb ? p[i] : 0.0;
    }
#pragma unroll
    for (int k = 0; k < kSumBatch; ++k) acc += v[k];
  }
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  if (lane == 0) *mean = (float)(acc / reduce_div);
}

// ------------------------------------------------------------------------------------------------
// fwl_wave_rows: one wavefront per row, C <= 64 * E (E elements per lane)

// Register rows: lane `lane` holds units lane + 64*k, k < NV, i.e. E = kUnit*NV elements in
// slots kUnit*k + e.
template <typename T, int NV, bool VEC>
__device__ __forceinline__ void load_row(rsrc_t row, int lane, float* x) {
  // all lanes load unconditionally; offsets past the row (or a zero-size resource: no row) read 0
#pragma unroll
  for (int k = 0; k < NV; ++k) load_unit<T, VEC>(row, (uint32_t)(lane + kWave * k), x + kUnit<T, VEC> * k);
}


// Line-aligned window of a row of 16-byte units from a 16-byte aligned start: the resource starts
// at the row's first 128-byte line boundary, `a` units (0..7) before the row, so every 1024-byte
// load of the wavefront covers exactly 8 lines (a row start inside a line makes it 9).  Lanes of
// the first load that fall in front of the row take an offset past the resource (they read 0,
// like lanes past the row's end); nothing outside the row is read.  a = 0 is plain addressing.
__device__ __forceinline__ uint32_t window_unit(int k, int lane, int a) {
  return k == 0 && lane < a ? (kOffNone >> 4) : (uint32_t)(lane + kWave * k);
}

template <typename T, int NV>
__device__ __forceinline__ void load_row_window(rsrc_t row, int lane, int a, float* x) {
#pragma unroll
  for (int k = 0; k < NV; ++k) load_unit<T, true>(row, window_unit(k, lane, a), x + kUnit<T, true> * k);
}

// element index of register slot i of this lane
template <typename T, bool VEC>
__device__ __forceinline__ int slot_index(int i, int lane) {
  constexpr int U = kUnit<T, VEC>;
  return U * (lane + kWave * (i / U)) + (i % U);
}


// element j of the register row (j wavefront-uniform, 0 <= j < C): the uniform slot index makes
// the register array access an indexed register move (s_set_gpr_idx), then one lane read
// (shift: units of the row's line-aligned window in front of its first element)
template <typename T, int NV, bool VEC>
__device__ __forceinline__ float element_at(const float* x, int j, int shift = 0) {
  constexpr int U = kUnit<T, VEC>;
  const int slot = uniform(U * ((j / U + shift) >> 6) + (j % U));
  const int owner = uniform((j / U + shift) & 63);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x[slot]), owner));
}

// exclusive prefix sum of v over the wavefront; `total` receives the sum of all lanes
__device__ __forceinline__ int wave_excl_scan_i32(int v, int& total) {
  int s = v;
  s += dpp_or0<0x111, 0xF>(s);          // row_shr:1
  s += dpp_or0<0x112, 0xF>(s);          // row_shr:2
  s += dpp_or0<0x114, 0xF>(s);          // row_shr:4
  s += dpp_or0<0x118, 0xF>(s);          // row_shr:8
  s += dpp_or0<kRowBcast15, 0xA>(s);
  s += dpp_or0<kRowBcast31, 0xC>(s);
  total = __builtin_amdgcn_readlane(s, 63);
  return s - v;
}


struct RowResult {
  float H;
  float loss;
  double l64;
  int kappa;
};

// The LDS candidate list of a wavefront holds up to a whole register row (E values per lane); the
// candidate-list mode keeps the element indices alongside.
constexpr int kRowsPerWave = kWave;   // rows of one wavefront per launch (labels/results: one lane each)

// Per-slot bias of a register row: -0.0 for slots inside the row, -inf past its end.  Slots past
// the end load 0, and x + bias sets them to -inf; for every other value x + (-0.0) == x (signed
// zeros included) except that a signaling NaN is quieted, so the result needs no further NaN
// quieting before max/min.
template <typename T, int NV, bool VEC>
__device__ __forceinline__ void row_bias(int C, int lane, float* bias) {
  constexpr int E = kUnit<T, VEC> * NV;
#pragma unroll
  for (int i = 0; i < E; ++i) bias[i] = slot_index<T, VEC>(i, lane) < C ? -0.0f : -INFINITY;
}

// fp64 sum and count of the register row's entries > thr, in a fixed order (slot order per lane,
// then the wavefront tree); the empty asm keeps the compiler from hoisting the conversions of the
// row out of the caller's loops (16-32 more VGPRs held across them)
template <int E>
__device__ __forceinline__ void reg_sum_count(const float* x, float thr, double& s, int& c) {
  double acc = 0.0;
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    float v = x[i];
    asm volatile("" : "+v"(v));
    const bool k = v > thr;
    acc += k ? (double)v : 0.0;
    cnt += k ? 1 : 0;
  }
  s = wave_sum_f64(acc);
  c = wave_sum_i32(cnt);
}

// the count alone (ballots on the scalar unit)
template <int E>
__device__ __forceinline__ int reg_count(const float* x, float thr) {
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) cnt += __popcll(ballot(x[i] > thr));
  return cnt;
}

// the same for bounds (see safe_lower32): per-lane fp32 partial sums added by an fp32 tree, the
// count from ballots (on the scalar unit, beside the tree's chain of dependent steps)
template <int E>
__device__ __forceinline__ void reg_sum_count32(const float* x, float thr, double& s, int& c) {
  static_assert(E <= 48, "safe_lower32 allows at most 48 values per lane with an fp32 tree");
  float acc = 0.0f;
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const bool k = x[i] > thr;
    acc += k ? x[i] : 0.0f;
    cnt += __popcll(ballot(k));
  }
  s = (double)wave_sum_f32(acc);
  c = cnt;
}

// A register row with more than 64 candidates z > t0 (its LDS list cl holds them, n of them;
// indices in ci_lds in candidate-list mode).  The tau of the 64 lane maxima, a subset of the row,
// is a lower bound t1 on tau, usually close to it.  At most 64 entries above t1 are staged again
// and sorted (resolve_list).  Otherwise fixed-point steps t <- H({z > t}) run over the registers:
// first with fp32 partial sums, each step a safe lower bound (safe_lower32), until they stall;
// then exact fp64 steps from there (each iterate <= tau, the set shrinking until it is the
// support), at most kRegSteps of them, and a bisection over the keys of (t1, m] after that, so
// that the passes over the registers are bounded.  The list keeps the candidates > t0 for the
// candidate-list output.
constexpr int kRegSteps = 32;
template <typename T, int MODE, int E, bool V4>
__device__ __forceinline__ void solve_many(const float* x, float lm, float t0, float m, int lane, float* cl,
                                           int* ci_lds, int& n, double& tau, int& kappa, uint64_t& support) {
  const double tl = select_tier<kWave>(lm, kWave, lane);
  float t1 = t0;
  if (tl == tl) {
    const float r = rd32(tl - ((double)kWave * (double)(fabsf(m) + 1.0f) + fabs(tl) + 1.0) * 0x1p-51);
    if (isfinite(r)) t1 = fmaxf(t0, prev_f32(r));
  }
  int n1 = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) n1 += __popcll(ballot(x[i] > t1));
  if (n1 <= kWave) {
    __builtin_amdgcn_wave_barrier();
    int at = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const bool c = x[i] > t1;
      const uint64_t b = ballot(c);
      if (b != 0) {
        if (c) {
          cl[at + rank_in(b)] = x[i];
          if constexpr (MODE == kCand) ci_lds[at + rank_in(b)] = slot_index<T, V4>(i, lane);
        }
        at += __popcll(b);
      }
    }
    n = n1;
    __builtin_amdgcn_wave_barrier();
    resolve_list(cl, n, t1, m, lane, tau, kappa, support);
    return;
  }
  support = 0;
  // bound steps with fp32 partial sums; the entries summed lie in (t, m], so their magnitudes are
  // at most max(|t|, |m|), which shrinks the allowance for rounding as t rises (rows of values
  // near 0 then take the steps until the set stops changing: fewer exact fp64 steps follow)
  float t = t1;
  for (int it = 0; it < kRegSteps; ++it) {
    double s;
    int c;
    reg_sum_count32<E>(x, t, s, c);
    const float nt = safe_lower32(s, c, fmaxf(fabsf(m), fabsf(t)));
    if (!(nt > t)) break;
    t = nt;
  }
  // exact steps from the bound
  double tt = (double)t, s;
  int c;
  reg_sum_count<E>(x, t, s, c);
  bool conv = false;
  tau = NAN;
  kappa = 0;
  for (int it = 0; it < kRegSteps && c > 0; ++it) {
    const double tn = (s - 1.0) / (double)c;
    // the set above the new iterate: its count decides, its fp64 sum is needed only for another
    // step (after bound steps that reached the support, the first step confirms it)
    const int c2 = reg_count<E>(x, rd32(tn));
    if (c2 == c || !(tn > tt)) {
      tau = tn;
      kappa = c2;
      conv = true;
      break;
    }
    double s2;
    reg_sum_count<E>(x, rd32(tn), s2, c);
    tt = tn;
    s = s2;
  }
  if (!conv) {
    // G(a) >= 1 > G(b) over keys: tau in [a, b), the support {z > a}
    int ka = fkey(t1 + 0.0f), kb = fkey(m + 0.0f);
    while ((int64_t)kb - ka > 1) {
      const int km = (int)(((int64_t)ka + kb) >> 1);
      const float v = fkey_inv(km);
      double s3;
      int c3;
      reg_sum_count<E>(x, v, s3, c3);
      if (s3 - (double)c3 * (double)v >= 1.0) ka = km;
      else kb = km;
    }
    double s3;
    int c3;
    reg_sum_count<E>(x, fkey_inv(ka), s3, c3);
    kappa = c3;
    tau = c3 > 0 ? (s3 - 1.0) / (double)c3 : NAN;
  }
  const double tc = clamp_below_max(tau, m);
  if (tc != tau) {
    double s3;
    tau = tc;
    reg_sum_count<E>(x, rd32(tau), s3, kappa);
  }
}

// One row: x holds it (E values per lane).  Once its candidates are in the LDS list, the loads of
// the next row (resource `next`, zero-size if there is none) are issued into xn, so they are in
// flight during the selection and the stores of this row; x stays for the outputs.
// AW: x and xn hold line-aligned windows (load_row_window), the current row `a` units into its
// window and the next row `an` units into its own; the gradient row shares the logits row's
// offset within its line.
template <typename T, int MODE, int NV, bool V4, bool AW>
__device__ __forceinline__ RowResult process_row(int64_t r, rsrc_t next, int64_t y64, int C, int lane,
                                                 float* x, float* xn, const float* bias, float* cl, int* ci_lds,
                                                 const Outs& o, int a, int an) {
  constexpr int U = kUnit<T, V4>;
  constexpr int E = U * NV;
  static_assert(std::is_same<T, float>::value || MODE != kMask, "16-bit logits: no mask output");
  static_assert(!AW || (std::is_same<T, float>::value && V4 && MODE == kGrad), "windows: fp32 gradient rows");
  const bool yok = y64 >= 0 && y64 < C;
  const int yr = yok ? (int)y64 : -1;
  if constexpr (AW) {
    // the row's units are a .. a + C/U - 1 of the window
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const float b = (uint32_t)(lane + kWave * k - a) < (uint32_t)(C / U) ? -0.0f : -INFINITY;
#pragma unroll
      for (int e = 0; e < U; ++e) x[U * k + e] += b;
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] += bias[i];
  }

  // row maximum and the first lower bound max - 1 (rounded down: every support entry passes)
  float lm = x[0];
#pragma unroll
  for (int i = 1; i < E; ++i) lm = fmaxf(lm, x[i]);
  const float m = wave_max_f32(lm);
  const float t0 = bound_below_max(m);

  // candidates z > t0, slot-major: the candidates of slot i follow those of the slots before it,
  // in lane order (slots without any candidate cost one compare)
  int n = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const bool c = x[i] > t0;
    const uint64_t b = ballot(c);
    if (b != 0) {
      if (c) {
        const int at = n + rank_in(b);
        cl[at] = x[i];
        if constexpr (MODE == kCand) ci_lds[at] = slot_index<T, V4>(i, lane);
      }
      n += __popcll(b);
    }
  }
  const float zy = yok ? element_at<T, NV, V4>(x, yr, AW ? a : 0) : NAN;
  __builtin_amdgcn_wave_barrier();
  if constexpr (AW) load_row_window<T, NV>(next, lane, an, xn);
  else load_row<T, NV, V4>(next, lane, xn);

  double tau;
  int kappa;
  uint64_t support;
  if (n <= kWave) resolve_list(cl, n, t0, m, lane, tau, kappa, support);
  else solve_many<T, MODE, E, V4>(x, lm, t0, m, lane, cl, ci_lds, n, tau, kappa, support);
  const float Hf = rd32(tau);
  __builtin_amdgcn_wave_barrier();

  const float inv = (float)(o.scale / (double)kappa);
  if constexpr (MODE == kGrad) {
    const int sh = AW ? a : 0;
    const rsrc_t out = make_rsrc(static_cast<char*>(o.grad) + r * (int64_t)C * kElemBytes<T> - 16 * sh,
                                 (uint32_t)(kElemBytes<T> * C + 16 * sh));
    const int qy = yr / U + sh, ky = yr >= 0 ? qy >> 6 : -1, ly = qy & 63, ey = yr % U;
    // the four values a gradient element can take, encoded once per row
    const uint32_t b_inv = encode<T>(inv), b_lab_in = encode<T>(inv - o.scale_f);
    const uint32_t b_lab_out = encode<T>(0.0f - o.scale_f);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      uint32_t g[U];
#pragma unroll
      for (int e = 0; e < U; ++e) g[e] = x[U * k + e] > Hf ? b_inv : 0u;
      if (k == ky && lane == ly) {
#pragma unroll
        for (int e = 0; e < U; ++e) g[e] = e == ey ? (x[U * k + e] > Hf ? b_lab_in : b_lab_out) : g[e];
      }
      store_unit_bits<T, V4>(out, AW ? window_unit(k, lane, a) : (uint32_t)(lane + kWave * k), g);
    }
  } else if constexpr (MODE == kMask) {
    const rsrc_t out = make_rsrc(o.mask + r * (int64_t)C, (uint32_t)C);
    if constexpr (V4) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const unsigned mk = (unsigned)(x[4 * k] > Hf) | ((unsigned)(x[4 * k + 1] > Hf) << 8) |
                            ((unsigned)(x[4 * k + 2] > Hf) << 16) | ((unsigned)(x[4 * k + 3] > Hf) << 24);
        __builtin_amdgcn_raw_buffer_store_b32(mk, out, 4 * (lane + kWave * k), 0, kNonTemporal);
      }
    } else {
#pragma unroll
      for (int k = 0; k < NV; ++k)
        __builtin_amdgcn_raw_buffer_store_b8((unsigned char)(x[k] > Hf), out, lane + kWave * k, 0, kNonTemporal);
    }
  } else {
    // the support list, in the (deterministic) order of the candidate list; lanes without an
    // entry store past the end of the resource (dropped)
    const rsrc_t outv = make_rsrc(o.cval + r * (int64_t)o.cstride, 4u * (uint32_t)o.ccap);
    const rsrc_t outi = make_rsrc(o.cidx + r * (int64_t)o.cstride, 4u * (uint32_t)o.ccap);
    int out = 0;
    for (int p0 = 0; p0 < n; p0 += kWave) {
      const int p = p0 + lane;
      const float v = p < n ? cl[p] : -INFINITY;
      const bool k = v > Hf;
      const uint64_t b = ballot(k);
      const uint32_t at = k ? 4u * (uint32_t)(out + rank_in(b)) : kOffNone;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), outv, at, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32((unsigned)(p < n ? ci_lds[p] : 0), outi, at, 0, 0);
      out += __popcll(b);
    }
  }
  __builtin_amdgcn_wave_barrier();

  RowResult res;
  res.H = Hf;
  res.l64 = (1.0 - (double)zy) + tau;
  res.loss = (float)res.l64;
  res.kappa = kappa;
  return res;
}

// Stores to a zero-size resource (dropped by the range check, no memory traffic), issued after the
// first row's loads so that the wait counts at the top of the row loop are the same on entry as on
// every later iteration (4 row loads followed by the row's stores); with a different mix on entry
// the compiler waits for every outstanding store at the top of each row.
template <typename T, int MODE, int NV, bool V4>
__device__ __forceinline__ void mirror_row_stores(int lane) {
  const rsrc_t none = make_rsrc(nullptr, 0u);
  if constexpr (MODE == kGrad) {
#pragma unroll
    for (int k = 0; k < NV; ++k) store_zero_unit<T, V4>(none, (uint32_t)(lane + kWave * k));
  } else if constexpr (MODE == kMask) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if constexpr (V4) __builtin_amdgcn_raw_buffer_store_b32(0u, none, 4 * (lane + kWave * k), 0, kNonTemporal);
      else __builtin_amdgcn_raw_buffer_store_b8((unsigned char)0, none, lane + kWave * k, 0, kNonTemporal);
    }
  }
}

// A wavefront handles rows w + k*stride, k < nrows <= 64.  Their labels arrive in one gather load
// before the first row, and their H, loss and kappa stay in registers (row k in lane k) until the
// last row, so the only memory instructions inside the row loop are the row loads and stores.
// AW: rows read and written through line-aligned windows (load_row_window); the host takes it for
// fp32 gradient rows of 16-byte multiples from 16-byte aligned logits and gradient that share their
// offsets within a 128-byte line.  A row whose window would not fit NV units per lane keeps plain
// addressing (shift 0).  16-bit rows keep plain addressing throughout: their kernel is issue-bound,
// and the per-row window arithmetic measured 4% slower there (bf16 65536 x 1000: 59.5 against
// 57.2 us; 65536 x 2000: 105.9 against 102.1).  Mask rows keep it too: windowed logits with the
// mask words shifted alike measured slower (65536 x 1000: 67.8 against 63.2 us).
template <typename T, int MODE, int NV, bool V4, bool AW>
__global__ __launch_bounds__(kBlock) void fwl_wave_rows(const void* __restrict__ z,
                                                        const int64_t* __restrict__ tgt, int64_t N,
                                                        int C, Outs o) {
  constexpr int E = kUnit<T, V4> * NV;
  constexpr int kListFloats = E * kWave;   // a whole register row
  constexpr int kIdx = MODE == kCand ? kListFloats : 1;
  __shared__ float s_list[kWavesPerBlock][kListFloats];
  __shared__ int s_idx[kWavesPerBlock][kIdx];
  __shared__ double s_wsum[kWavesPerBlock];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  const int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wid;   // this wavefront's rows: w + k*stride
  const int nrows = w < N ? (int)((N - 1 - w) / stride + 1) : 0;   // <= kRowsPerWave (host grid)
  const uint32_t row_bytes = (uint32_t)(kElemBytes<T> * C);
  // units of row k's window in front of the row (0 without windows, or where the window would
  // not fit the lanes' NV units)
  const int fit = kWave * NV - (C + kUnit<T, V4> - 1) / kUnit<T, V4>;
  auto row_shift = [&](int k) {
    if constexpr (!AW) return 0;
    const uintptr_t p = reinterpret_cast<uintptr_t>(z) + (uintptr_t)((w + (int64_t)k * stride) * o.ld * kElemBytes<T>);
    const int a = (int)((p >> 4) & 7);
    return k < nrows && a <= fit ? uniform(a) : 0;
  };
  auto row_rsrc = [&](int k) {
    const int sh = row_shift(k);
    return k < nrows ? make_rsrc(static_cast<const char*>(z) + (w + (int64_t)k * stride) * o.ld * kElemBytes<T> - 16 * sh,
                                 row_bytes + 16u * (uint32_t)sh)
                     : make_rsrc(z, 0u);
  };
  const int64_t my_y = lane < nrows ? tgt[w + (int64_t)lane * stride] : 0;
  float my_H = 0.0f, my_loss = 0.0f;
  double my_l64 = 0.0;
  int my_kappa = 0;
  double lsum = 0.0;
  float xa[E], xb[E], bias[E];
  if constexpr (!AW) row_bias<T, NV, V4>(C, lane, bias);
  auto row = [&](int k, float* x, float* xn) {
    const int64_t y = ((int64_t)__builtin_amdgcn_readlane((int)(my_y >> 32), k) << 32) |
                      (uint32_t)__builtin_amdgcn_readlane((int)my_y, k);
    const RowResult res = process_row<T, MODE, NV, V4, AW>(w + (int64_t)k * stride, row_rsrc(k + 1), y, C, lane, x,
                                                        xn, bias, s_list[wid], s_idx[wid], o, row_shift(k),
                                                        row_shift(k + 1));
    lsum += (double)res.loss;
    if (lane == k) {
      my_H = res.H;
      my_loss = res.loss;
      my_l64 = res.l64;
      my_kappa = res.kappa;
    }
  };
  if (nrows > 0) {
    if constexpr (AW) load_row_window<T, NV>(row_rsrc(0), lane, row_shift(0), xa);
    else load_row<T, NV, V4>(row_rsrc(0), lane, xa);
    __builtin_amdgcn_sched_barrier(0);   // keep the mirror stores after the loads
    mirror_row_stores<T, MODE, NV, V4>(lane);
    __builtin_amdgcn_sched_barrier(0);
    // two row buffers whose roles alternate: the loop is unrolled by two so that no buffer is copied
    int k = 0;
    while (true) {
      row(k, xa, xb);
      if (++k >= nrows) break;
      row(k, xb, xa);
      if (++k >= nrows) break;
    }
  }
  if (lane < nrows) {
    const int64_t r = w + (int64_t)lane * stride;
    if (o.H) o.H[r] = my_H;
    if (o.loss) o.loss[r] = my_loss;
    if (o.loss64) o.loss64[r] = my_l64;
    if (o.kappa) o.kappa[r] = my_kappa;
    if constexpr (MODE == kCand) o.ccnt[r] = my_kappa;
  }
  if (lane == 0) s_wsum[wid] = lsum;
  __syncthreads();
  const double bsum = (s_wsum[0] + s_wsum[1]) + (s_wsum[2] + s_wsum[3]);
  mean_epilogue(bsum, o);
}

// ------------------------------------------------------------------------------------------------
// fwl_seg_rows: short rows, R = 64/L rows per wavefront iteration, one row per aligned group
// ("segment") of L = 16 or 32 lanes.  Every cross-lane step of fwl_wave_rows works inside the
// segments at once (DPP within rows of 16 lanes, v_permlane16_swap between the two rows of a
// 32-lane segment), so R rows share each instruction of the selection.

// butterfly reductions inside segments: every lane receives its segment's result
template <int L>
__device__ __forceinline__ float seg_max_f32(float v, int lane) {
  v = fmaxf(v, xor_lane<1>(v, lane));
  v = fmaxf(v, xor_lane<2>(v, lane));
  v = fmaxf(v, __int_as_float(dpp_mov<kRowHalfMirror>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<kRowMirror>(__float_as_int(v))));
  if constexpr (L == 32) v = fmaxf(v, xor_lane<16>(v, lane));
  return v;
}

template <int L>
__device__ __forceinline__ double seg_max_f64(double v, int lane) {
  v = fmax(v, dpp_mov_f64<kQuadXor1>(v));
  v = fmax(v, dpp_mov_f64<kQuadXor2>(v));
  v = fmax(v, dpp_mov_f64<kRowHalfMirror>(v));
  v = fmax(v, dpp_mov_f64<kRowMirror>(v));
  if constexpr (L == 32) {
    const int64_t b = __double_as_longlong(v);
    const float lo = xor_lane<16>(__int_as_float((int)b), lane);
    const float hi = xor_lane<16>(__int_as_float((int)(b >> 32)), lane);
    v = fmax(v, __longlong_as_double((int64_t)(((uint64_t)(unsigned)__float_as_int(hi) << 32) |
                                               (unsigned)__float_as_int(lo))));
  }
  return v;
}

// (all lanes of a segment get bit-identical sums: every butterfly step adds two commuted operands)
template <int L>
__device__ __forceinline__ double seg_sum_f64(double v, int lane) {
  v += dpp_mov_f64<kQuadXor1>(v);
  v += dpp_mov_f64<kQuadXor2>(v);
  v += dpp_mov_f64<kRowHalfMirror>(v);
  v += dpp_mov_f64<kRowMirror>(v);
  if constexpr (L == 32) {
    const int64_t b = __double_as_longlong(v);
    const float lo = xor_lane<16>(__int_as_float((int)b), lane);
    const float hi = xor_lane<16>(__int_as_float((int)(b >> 32)), lane);
    v += __longlong_as_double((int64_t)(((uint64_t)(unsigned)__float_as_int(hi) << 32) |
                                        (unsigned)__float_as_int(lo)));
  }
  return v;
}

template <int L>
__device__ __forceinline__ int seg_sum_i32(int v, int lane) {
  v += dpp_mov<kQuadXor1>(v);
  v += dpp_mov<kQuadXor2>(v);
  v += dpp_mov<kRowHalfMirror>(v);
  v += dpp_mov<kRowMirror>(v);
  if constexpr (L == 32) v += __float_as_int(xor_lane<16>(__int_as_float(v), lane));
  return v;
}

// exclusive prefix sum inside segments
template <int L>
__device__ __forceinline__ int seg_excl_scan_i32(int v) {
  int s = v;
  s += dpp_or0<0x111, 0xF>(s);   // row_shr:1
  s += dpp_or0<0x112, 0xF>(s);   // row_shr:2
  s += dpp_or0<0x114, 0xF>(s);   // row_shr:4
  s += dpp_or0<0x118, 0xF>(s);   // row_shr:8
  if constexpr (L == 32) s += dpp_or0<kRowBcast15, 0xA>(s);   // rows 1, 3 += last lane of rows 0, 2
  return s - v;
}

// bitonic sort of every segment, descending: stages below L alternate direction by lane bit K,
// the last stage sorts every segment descending
constexpr uint64_t seg_keep_max_mask(int K, int J, int L) {
  uint64_t m = 0;
  for (int i = 0; i < 64; ++i) {
    const bool desc = K >= L || (i & K) == 0;
    if (((i & J) == 0) == desc) m |= 1ull << i;
  }
  return m;
}

template <int K, int J, int L>
__device__ __forceinline__ float seg_bitonic_step(float v, int lane) {
  const float p = xor_lane<J>(v, lane);
  return select_lanes(seg_keep_max_mask(K, J, L), fmaxf(v, p), fminf(v, p));
}

template <int K, int L>
__device__ __forceinline__ float seg_bitonic_merge(float v, int lane) {
  if constexpr (K >= 32) v = seg_bitonic_step<K, 16, L>(v, lane);
  if constexpr (K >= 16) v = seg_bitonic_step<K, 8, L>(v, lane);
  if constexpr (K >= 8) v = seg_bitonic_step<K, 4, L>(v, lane);
  if constexpr (K >= 4) v = seg_bitonic_step<K, 2, L>(v, lane);
  return seg_bitonic_step<K, 1, L>(v, lane);
}

template <int L>
__device__ __forceinline__ float seg_sort_desc(float v, int lane) {
  v = seg_bitonic_merge<2, L>(v, lane);
  v = seg_bitonic_merge<4, L>(v, lane);
  v = seg_bitonic_merge<8, L>(v, lane);
  v = seg_bitonic_merge<16, L>(v, lane);
  if constexpr (L == 32) v = seg_bitonic_merge<32, L>(v, lane);
  return v;
}

template <int K, int J, int L>
__device__ __forceinline__ int seg_bitonic_step_i(int v, int lane) {
  const int p = xor_lane_i<J>(v, lane);
  return select_lanes_i(seg_keep_max_mask(K, J, L), max(v, p), min(v, p));
}

template <int K, int L>
__device__ __forceinline__ int seg_bitonic_merge_i(int v, int lane) {
  if constexpr (K >= 32) v = seg_bitonic_step_i<K, 16, L>(v, lane);
  if constexpr (K >= 16) v = seg_bitonic_step_i<K, 8, L>(v, lane);
  if constexpr (K >= 8) v = seg_bitonic_step_i<K, 4, L>(v, lane);
  if constexpr (K >= 4) v = seg_bitonic_step_i<K, 2, L>(v, lane);
  return seg_bitonic_step_i<K, 1, L>(v, lane);
}

// integer keys (fkey) of every segment sorted descending
template <int L>
__device__ __forceinline__ int seg_sort_desc_i(int v, int lane) {
  v = seg_bitonic_merge_i<2, L>(v, lane);
  v = seg_bitonic_merge_i<4, L>(v, lane);
  v = seg_bitonic_merge_i<8, L>(v, lane);
  v = seg_bitonic_merge_i<16, L>(v, lane);
  if constexpr (L == 32) v = seg_bitonic_merge_i<32, L>(v, lane);
  return v;
}

// value of lane src (per-lane source) through the LDS crossbar
__device__ __forceinline__ double bpermute_f64(int src, double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_ds_bpermute(4 * src, (int)b);
  const int hi = __builtin_amdgcn_ds_bpermute(4 * src, (int)(b >> 32));
  return __longlong_as_double((int64_t)(((uint64_t)(unsigned)hi << 32) | (unsigned)lo));
}

// sum/count of the entries > thr among the first n of one segment's list (li = lane in segment;
// nmax = the largest n of the wavefront's segments)
template <int L>
__device__ __forceinline__ void seg_list_sum_count(const float* cl, int n, int nmax, float thr, int li, int lane,
                                                   double& s, int& c) {
  double acc = 0.0;
  int cnt = 0;
  for (int p0 = 0; p0 < nmax; p0 += L) {
    const int p = p0 + li;
    const float v = p < n ? cl[p] : -INFINITY;
    const bool k = v > thr;
    acc += k ? (double)v : 0.0;
    cnt += k ? 1 : 0;
  }
  s = seg_sum_f64<L>(acc, lane);
  c = seg_sum_i32<L>(cnt, lane);
}

// one element (for z_y): unit-agnostic 32/16-bit buffer load at element offset j
template <typename T>
__device__ __forceinline__ float load_one(rsrc_t r, uint32_t byte_off) {
  if constexpr (std::is_same<T, float>::value)
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
  else
    return widen16<T>(__builtin_amdgcn_raw_buffer_load_b16(r, byte_off, 0, 0));
}


// A wavefront handles groups g = w + k*stride of R consecutive rows (rows g*R + s, s < R); lane j
// holds the label of the wavefront's row j = k*R + s.  The group's rows share one buffer resource;
// units past a row's end are masked on load and dropped on store.  Two register buffers alternate
// (the loop is unrolled by two): the next group loads into one while the other is resolved and
// its outputs are computed from the values.
template <typename T, int MODE, int L, int NV, bool V4>
__global__ __launch_bounds__(kBlock) void fwl_seg_rows(const void* __restrict__ z,
                                                       const int64_t* __restrict__ tgt, int64_t N, int C,
                                                       Outs o) {
  constexpr int R = kWave / L;
  constexpr int U = kUnit<T, V4>;
  constexpr int E = U * NV;
  constexpr unsigned kSegMask = L == 32 ? 0xFFFFFFFFu : 0xFFFFu;
  static_assert(E <= 32, "one mask bit per register slot");
  static_assert(MODE != kCand, "candidate lists: fwl_wave_rows");
  static_assert(std::is_same<T, float>::value || MODE == kGrad, "16-bit logits: fused op only");
  __shared__ float s_list[kWavesPerBlock][E * kWave];
  __shared__ double s_wsum[kWavesPerBlock];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int seg = lane / L;          // segment of this lane
  const int li = lane % L;           // lane within the segment
  float* cl = s_list[wid];
  const int64_t G = (N + R - 1) / R;                        // row groups
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  const int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wid;
  const int ngroups = w < G ? (int)((G - 1 - w) / stride + 1) : 0;   // <= kWave / R (host grid)
  const uint32_t row_bytes = (uint32_t)(kElemBytes<T> * C);
  const uint32_t ld_bytes = (uint32_t)(kElemBytes<T> * o.ld);   // logits row stride (>= row_bytes)
  const int units_row = C / U;                               // V4 rows: C and ld are multiples of U
  auto group_rows = [&](int k) -> int {
    const int64_t r0 = (w + (int64_t)k * stride) * R;
    return k < ngroups ? (int)(N - r0 < R ? N - r0 : R) : 0;
  };
  auto group_rsrc = [&](int k) {
    const int rows = group_rows(k);
    const char* base = static_cast<const char*>(z) + (w + (int64_t)(k < ngroups ? k : 0) * stride) * R * (int64_t)ld_bytes;
    return make_rsrc(base, rows > 0 ? (uint32_t)(rows - 1) * ld_bytes + row_bytes : 0u);
  };
  int64_t my_y = 0;
  {
    const int kk = lane / R, ss = lane % R;
    const int64_t r = (w + (int64_t)kk * stride) * R + ss;
    if (kk < ngroups && r < N) my_y = tgt[r];
  }
  auto seg_label = [&](int k) -> int64_t {   // label of this lane's segment row in group k
    const int src = (k * R + seg) & 63;
    const int lo = __builtin_amdgcn_ds_bpermute(4 * src, (int)my_y);
    const int hi = __builtin_amdgcn_ds_bpermute(4 * src, (int)(my_y >> 32));
    return (int64_t)(((uint64_t)(unsigned)hi << 32) | (unsigned)lo);
  };
  auto label_off = [&](int64_t y) -> uint32_t {
    return (y >= 0 && y < C) ? (uint32_t)seg * ld_bytes + (uint32_t)(y * kElemBytes<T>) : kOffNone;
  };
  double lsum = 0.0;   // losses of the rows whose results this lane (a segment's lane 0) wrote
  float xa[E], xb[E], bias[E];
  // -0.0 inside the row, -inf past its end (see row_bias)
#pragma unroll
  for (int i = 0; i < E; ++i) bias[i] = li + L * (i / U) < units_row ? -0.0f : -INFINITY;
  auto load_group = [&](rsrc_t rs, float* xx) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = li + L * k;
      load_unit<T, V4>(rs, u < units_row ? (uint32_t)(seg * (ld_bytes / (U * kElemBytes<T>)) + u) : (kOffNone >> 4),
                       xx + U * k);
    }
  };
  float zy_next = 0.0f;
  auto group = [&](int k, float* x, float* xn) {
    const int rows = group_rows(k);
    const int64_t y64 = seg_label(k);
    const bool yok = y64 >= 0 && y64 < C;
    const int yr = yok ? (int)y64 : -1;
    const float zy = zy_next;
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] += bias[i];
    if (rows < R) {   // phantom segments of a short last group
      const bool valid = seg < rows;
#pragma unroll
      for (int i = 0; i < E; ++i) x[i] = valid ? x[i] : -INFINITY;
    }
    float lm = x[0];
#pragma unroll
    for (int i = 1; i < E; ++i) lm = fmaxf(lm, x[i]);
    const float m = seg_max_f32<L>(lm, lane);
    const float t0 = bound_below_max(m);
    // candidates z > t0, lane-major inside the segment's list
    unsigned cm = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) cm |= (unsigned)(x[i] > t0) << i;
    const int cnt = __popc(cm);
    const int base = seg_excl_scan_i32<L>(cnt);
    const int n = seg_sum_i32<L>(cnt, lane);
    float* cls = cl + seg * (L * E);   // this segment's list
    {
      int pos = base;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        if ((cm >> i) & 1u) {
          cls[pos] = x[i];
          ++pos;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    // next group's loads into the other buffer
    const bool has_next = k + 1 < ngroups;
    const rsrc_t rs_next = has_next ? group_rsrc(k + 1) : make_rsrc(z, 0u);
    load_group(rs_next, xn);
    zy_next = load_one<T>(rs_next, label_off(seg_label(has_next ? k + 1 : k)));

    double tau = NAN;
    int kappa = 0;
    const bool big = ballot(n > L) != 0;
    if (!big) {
      // sort, fp64 prefix sums, the support size by k z_(k) > S_k - 1 (see select_tier)
      const float c = li < n ? cls[li] : -INFINITY;
      int key = fkey(li < n ? c + 0.0f : -INFINITY);
      key = seg_sort_desc_i<L>(key, lane);
      const float v = fkey_inv(key);
      const double S = scan_f64<L>(li < n ? (double)v : 0.0);
      const uint64_t in = ballot(li < n && (double)v * (double)(li + 1) > S - 1.0);
      const unsigned sb = ((unsigned)(in >> (seg * L)) & kSegMask) | 1u;
      const int kap = 32 - __clz(sb);
      const double Sk = bpermute_f64(seg * L + kap - 1, S);
      tau = n > 0 ? clamp_below_max((Sk - 1.0) / (double)kap, m) : NAN;
      const uint64_t sup = ballot(li < n && c > rd32(tau));
      kappa = __popc((unsigned)(sup >> (seg * L)) & kSegMask);
    } else {
      // fixed-point iterations per segment over its list, until every segment has converged
      const int nmax = (int)wave_max_f32((float)n);
      double t = (double)t0, s, s2;
      int c, c2;
      seg_list_sum_count<L>(cls, n, nmax, t0, li, lane, s, c);
      bool done = n == 0;
      for (int it = 0; it <= nmax + 1; ++it) {
        if (ballot(!done) == 0) break;
        const double tn = (s - 1.0) / (double)c;
        seg_list_sum_count<L>(cls, n, nmax, rd32(tn), li, lane, s2, c2);
        if (!done) {
          if (c2 == c || !(tn > t)) {
            tau = tn;
            kappa = c2;
            done = true;
          } else {
            t = tn;
            s = s2;
            c = c2;
          }
        }
      }
      const double tc = n > 0 ? clamp_below_max(tau, m) : tau;
      const bool clamped = tc != tau && n > 0;
      if (ballot(clamped) != 0) {
        double s3;
        int k3;
        seg_list_sum_count<L>(cls, n, nmax, rd32(tc), li, lane, s3, k3);
        if (clamped) kappa = k3;
      }
      tau = tc;
    }
    __builtin_amdgcn_wave_barrier();
    const float Hf = rd32(tau);
    const float inv = (float)(o.scale / (double)kappa);
    const int64_t row0 = (w + (int64_t)k * stride) * R;   // first row of this group
    const int qy = yr / U, ky = yr >= 0 ? qy / L : -1, lyl = qy % L, ey = yr % U;
    if constexpr (MODE == kGrad) {
      const rsrc_t outr = make_rsrc(static_cast<char*>(o.grad) + row0 * (int64_t)row_bytes,
                                    (uint32_t)rows * row_bytes);
      const uint32_t b_inv = encode<T>(inv), b_lab_in = encode<T>(inv - o.scale_f);
      const uint32_t b_lab_out = encode<T>(0.0f - o.scale_f);
#pragma unroll
      for (int kk = 0; kk < NV; ++kk) {
        const int u = li + L * kk;
        uint32_t g[U];
#pragma unroll
        for (int e = 0; e < U; ++e) g[e] = x[U * kk + e] > Hf ? b_inv : 0u;
        if (kk == ky && li == lyl) {
#pragma unroll
          for (int e = 0; e < U; ++e) g[e] = e == ey ? (x[U * kk + e] > Hf ? b_lab_in : b_lab_out) : g[e];
        }
        store_unit_bits<T, V4>(outr, u < units_row ? (uint32_t)(seg * units_row + u) : (kOffNone >> 4), g);
      }
    } else {
      const rsrc_t outr = make_rsrc(o.mask + row0 * (int64_t)C, (uint32_t)(rows * C));
#pragma unroll
      for (int kk = 0; kk < NV; ++kk) {
        const int u = li + L * kk;
        if constexpr (V4) {
          const unsigned mk = (unsigned)(x[4 * kk] > Hf) | ((unsigned)(x[4 * kk + 1] > Hf) << 8) |
                              ((unsigned)(x[4 * kk + 2] > Hf) << 16) | ((unsigned)(x[4 * kk + 3] > Hf) << 24);
          __builtin_amdgcn_raw_buffer_store_b32(mk, outr, u < units_row ? (uint32_t)(seg * C + 4 * u) : kOffNone, 0,
                                                kNonTemporal);
        } else {
          __builtin_amdgcn_raw_buffer_store_b8((unsigned char)(x[kk] > Hf), outr,
                                               u < units_row ? (uint32_t)(seg * C + u) : kOffNone, 0, kNonTemporal);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    // per-row results, written by lane 0 of each segment
    if (li == 0 && seg < rows) {
      const double l64 = (1.0 - (double)(yok ? zy : NAN)) + tau;
      const float loss = (float)l64;
      const int64_t r = row0 + seg;
      if (o.H) o.H[r] = Hf;
      if (o.loss) o.loss[r] = loss;
      if (o.loss64) o.loss64[r] = l64;
      if (o.kappa) o.kappa[r] = kappa;
      lsum += (double)loss;
    }
  };
  if (ngroups > 0) {
    rsrc_t rs = group_rsrc(0);
    load_group(rs, xa);
    zy_next = load_one<T>(rs, label_off(seg_label(0)));
    __builtin_amdgcn_sched_barrier(0);   // mirror of the loop's stores (see mirror_row_stores)
    {
      const rsrc_t none = make_rsrc(nullptr, 0u);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if constexpr (MODE == kGrad) store_zero_unit<T, V4>(none, (uint32_t)(li + L * k));
        else if constexpr (V4) __builtin_amdgcn_raw_buffer_store_b32(0u, none, 4u * (uint32_t)(li + L * k), 0, kNonTemporal);
        else __builtin_amdgcn_raw_buffer_store_b8((unsigned char)0, none, (uint32_t)(li + L * k), 0, kNonTemporal);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    int k = 0;
    while (true) {
      group(k, xa, xb);
      if (++k >= ngroups) break;
      group(k, xb, xa);
      if (++k >= ngroups) break;
    }
  }
  const double wsum = wave_sum_f64(lsum);
  if (lane == 0) s_wsum[wid] = wsum;
  __syncthreads();
  const double bsum = (s_wsum[0] + s_wsum[1]) + (s_wsum[2] + s_wsum[3]);
  mean_epilogue(bsum, o);
}

// ------------------------------------------------------------------------------------------------
// fwl_block_rows: one block per row, streaming with LDS candidate lists

constexpr int kHistBlock = 1024;    // bins of a block's histogram (select_in_memory, W = 4)
constexpr int kTightenSteps = 2;    // fixed-point steps per tightening of a candidate list (fastest at sigma 0.001-0.1: 1, 2, 4, 12 measured)

// LDS of the block kernels.  While a row streams, each wavefront keeps its candidate list (value,
// index) in bval/bidx; the overflow solve (select_in_memory) reuses the same bytes, first as a
// histogram, then as one list of values.
struct alignas(16) BlockShared {
  union {
    struct {
      float bval[kWavesPerBlock][kCapMax];
      int bidx[kWavesPerBlock][kCapMax];
    };
    struct {
      unsigned hcnt[kHistBlock];
      double hsum[kHistBlock];
    };
    float blist[2 * kWavesPerBlock * kCapMax];
  };
  float trash[kWavesPerBlock][kWave];   // each lane's sink for the list appends it does not make
  float sel[kWave];
  float wmax[kWavesPerBlock];
  float wlo[kWavesPerBlock];      // each wavefront's lower bound on tau
  float wB[kWavesPerBlock];       // bound on the magnitude of the entries summed for wlo
  int wn[kWavesPerBlock];
  int wsel[kWavesPerBlock];
  int ovf[kWavesPerBlock];
  double red_s[kWavesPerBlock];
  int red_c[kWavesPerBlock];
  int wnx[kWavesPerBlock];         // the wavefront's list outgrew its indices (long lists only)
  uint64_t defm[kWavesPerBlock];   // fwl_overflow_rows: the deferred rows among the next kBlock
  int ncol;
  double tau;
  int kappa;
};
static_assert(sizeof(unsigned) * kHistBlock + sizeof(double) * kHistBlock <= 8 * kWavesPerBlock * kCapMax,
              "the histogram reuses the candidate lists");

// The list of one wavefront of fwl_wave_stream_rows: up to kWaveVCap candidate values, the first
// kCapMax of them with their indices, which live in the list's last kCapMax slots while the list
// holds at most kCapMax entries.  A row whose list outgrows the indices keeps its values (tau
// comes from them) and writes its support from one more pass over the row (the two-pass op's
// write pass): rows of low-variance logits (hundreds to thousands of support entries) then need
// no overflow solve.  49 KB of LDS per block (lists and trash slots): three blocks per CU.
// The two-pass op's read pass holds kStreamVCapLong values per list (66.5 KB per block, two
// blocks per CU, enough for one row per wavefront at 2048 rows of the chip's 256 CUs): a list
// that is full before its row ends is tightened, and at N(0, 0.001^2) rows of 131072 elements
// (supports of about 2700) a 3072-value list took about 11 tightenings per row, a 4096-value one
// about 5 (2048 x 131072: 607 -> 582 us per step; 4864 values: no better).
constexpr int kWaveVCap = 3072;
constexpr int kStreamVCapLong = 4096;
static_assert(kWaveVCap >= 2 * kCapMax && kWaveVCap % (4 * kWave) == 0, "indices share the value list");
static_assert(kStreamVCapLong >= 2 * kCapMax && kStreamVCapLong % (4 * kWave) == 0, "indices share the value list");
template <int CAP>
struct alignas(16) WaveShared {
  float val[CAP];
  float trash[kWave];   // each lane's sink for the list appends it does not make
};

// fwl_block_rows with long lists (the two-pass op's read pass on few rows): each wavefront's list
// holds kWaveVCap values, the first kCapMax with their indices in the list's last kCapMax slots
// (as in fwl_wave_stream_rows); 48 KB of lists per block.
struct alignas(16) BlockSharedBig {
  union {
    float bval[kWavesPerBlock][kWaveVCap];
    struct {
      unsigned hcnt[kHistBlock];
      double hsum[kHistBlock];
    };
    float blist[2 * kWavesPerBlock * kCapMax];
  };
  float trash[kWavesPerBlock][kWave];
  float sel[kWave];
  float wmax[kWavesPerBlock];
  float wlo[kWavesPerBlock];
  float wB[kWavesPerBlock];
  int wn[kWavesPerBlock];
  int wsel[kWavesPerBlock];
  int ovf[kWavesPerBlock];
  int wnx[kWavesPerBlock];         // the wavefront's list outgrew its indices
  double red_s[kWavesPerBlock];
  int red_c[kWavesPerBlock];
  int ncol;
  double tau;
  int kappa;
};

// Streaming rounds.  A row is shared by W wavefronts (W = 4: one block per row; W = 1: one
// wavefront per row).  In round `round`, access group u of a lane covers unit
//     (W > 1 ? wid*64 : 0) + lane + 64*W*(round*PER + u)
// where a unit is kUnit<T, VEC> elements (a 128-bit access, PER = kStreamUnroll groups per round)
// or a single element (PER = kRoundSlotsV1); slot kUnit*u + e holds element kUnit*unit + e.
template <int W, int PER>
__device__ __forceinline__ int lane_unit(int round, int u, int wid, int lane) {
  return (W > 1 ? wid * kWave : 0) + lane + kWave * W * (round * PER + u);
}

template <typename T, bool VEC>
struct Round {
  static constexpr int kPer = VEC ? kStreamUnroll : kRoundSlotsV1;   // access groups per round
  static constexpr int kSlots = kUnit<T, VEC> * kPer;
  float x[kSlots];
};

template <int W, typename T, bool VEC>
__device__ __forceinline__ int round_slot_index(int round, int slot, int wid, int lane) {
  constexpr int U = kUnit<T, VEC>;
  return U * lane_unit<W, Round<T, VEC>::kPer>(round, slot / U, wid, lane) + (slot % U);
}

// loads of one round, unconditional: offsets past the row read 0 (masked to -inf when used)
template <int W, typename T, bool VEC>
__device__ __forceinline__ void load_round(rsrc_t row, int round, int wid, int lane, Round<T, VEC>& a) {
  constexpr int PER = Round<T, VEC>::kPer;
#pragma unroll
  for (int u = 0; u < PER; ++u)
    load_unit<T, VEC>(row, (uint32_t)lane_unit<W, PER>(round, u, wid, lane), a.x + kUnit<T, VEC> * u);
}

// zero placeholders for every output element of one round (support entries are rewritten at
// the end of the row); offsets past the row end are dropped by the range check
template <int W, typename T, int MODE, bool VEC>
__device__ __forceinline__ void zero_round(rsrc_t out, int round, int wid, int lane) {
  constexpr int PER = Round<T, VEC>::kPer;
  if constexpr (MODE == kGrad) {
#pragma unroll
    for (int u = 0; u < PER; ++u) store_zero_unit<T, VEC>(out, (uint32_t)lane_unit<W, PER>(round, u, wid, lane));
  } else if constexpr (MODE == kMask) {
    // float rows only: one mask byte per element
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const uint32_t q = (uint32_t)lane_unit<W, PER>(round, u, wid, lane);
      if constexpr (VEC) __builtin_amdgcn_raw_buffer_store_b32(0u, out, 4u * q, 0, kNonTemporal);
      else __builtin_amdgcn_raw_buffer_store_b8((unsigned char)0, out, q, 0, kNonTemporal);
    }
  }
}

// One wavefront's state while a row (or a stretch of one) streams.
struct StreamState {
  int n;          // entries in the wavefront's list: every entry seen so far that is > t
  bool noidx;     // the list outgrew its indices: values only from then on
  float m;        // running maximum
  float t;        // running lower bound on tau
  bool ovf;       // the list could not hold the entries > t; from then on the scan only sums
  float tov;      // the bound at the overflow: acc_s/acc_c hold the entries > tov seen since
  double acc_s;   // (per lane)
  int acc_c;      // (per lane)
  int ylab;       // an element index of the span whose value is kept in zy as it streams by (-1: none)
  float zy;
  int sh;         // elements of the streamed window in front of the row (a window that starts on a
                  // 4-byte boundary before a 16-bit row of odd start; 0 otherwise)
};

__device__ __forceinline__ StreamState stream_state(bool force) {
  StreamState st;
  st.n = 0;
  st.noidx = false;
  st.m = -INFINITY;
  st.t = -INFINITY;
  st.ovf = force;   // forced: no list, only the sums (the overflow solve's path for every row)
  st.tov = NAN;     // set at the overflow (forced: at the first round)
  st.acc_s = 0.0;
  st.acc_c = 0;
  st.ylab = -1;
  st.zy = NAN;
  st.sh = 0;
  return st;
}

// Raise the wavefront's lower bound t with fixed-point steps t <- H({entries > t}) over its list
// and the round held in registers (a subset of the row, so H of it is <= tau), then drop the list
// entries <= the last step's start (not in the support: their output stays the zero written while
// streaming).  The last step's sum comes from the compaction itself, so the list may keep entries
// in (that start, t]: every reader of a list filters by its bound.
// The list (bv, and bi unless noidx) is padded storage (pad_list): at most 64 entries per lane,
// so its fp32 partial sums stay within what safe_lower32 allows.
template <int S>
__device__ __forceinline__ void tighten(float* bv, int* bi, int& n, float& t, const float* x, float m, bool noidx,
                                       int lane) {
  const float B = fmaxf(fabsf(m), fabsf(t));
  pad_list(bv, n, lane);
  auto round_part = [&](float thr, float& rs, int& rc) {
    rs = 0.0f;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const bool k = x[i] > thr;
      rs += k ? x[i] : 0.0f;
      rc += k ? 1 : 0;
    }
  };
  float tf = t;
  for (int it = 0; it + 1 < kTightenSteps; ++it) {
    // per-lane fp32 partial sums of the list and of the round (a bound needs no exact sum)
    float ls, rs;
    int lc;
    list4_lane<float>(bv, n, tf, lane, ls, lc);
    round_part(tf, rs, lc);
    const float nt = safe_lower32(wave_sum_f64((double)ls + (double)rs), wave_sum_i32(lc), B);
    if (!(nt > tf)) break;
    tf = nt;
  }
  float ks, rs;
  int kc;
  n = list4_compact_sum(bv, bi, n, tf, noidx, lane, ks, kc);
  round_part(tf, rs, kc);
  const float nt = safe_lower32(wave_sum_f64((double)ks + (double)rs), wave_sum_i32(kc), B);
  t = fmaxf(t, fmaxf(tf, nt));
}

// Candidates of one round: the running maximum m gives the bound t (>= m - 1 rounded down), and
// the entries z > t are appended to the wavefront's list.  A round whose entries do not fit is
// first used to tighten t; if they still do not fit, the list is abandoned: from then on the
// entries above the bound of that moment (tov) are only summed (their H is a lower bound on tau
// for the overflow solve).
// (cap: the list's capacity in values; icap <= cap: entries that keep their indices)
//
template <int W, typename T, bool VEC>
__device__ __forceinline__ void scan_round(Round<T, VEC>& a, int round, int C, int wid, int lane, float* bv,
                                           int* bi, float* tr, int cap, int icap, StreamState& st) {
  constexpr int S = Round<T, VEC>::kSlots;
  constexpr int kRoundElems = kUnit<T, VEC> * kWave * W * Round<T, VEC>::kPer;
  if (st.ylab >= round * kRoundElems && st.ylab < (round + 1) * kRoundElems) {
    // the round that holds element ylab: its value, from the lane that has it
    float v = 0.0f;
    bool f = false;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const bool h = round_slot_index<W, T, VEC>(round, i, wid, lane) == st.ylab;
      v = h ? a.x[i] : v;
      f = f || h;
    }
    const uint64_t b = ballot(f);
    if (b != 0) st.zy = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)__builtin_ctzll(b)));
  }
  float lm = -INFINITY;
  if ((round + 1) * kRoundElems <= C && (round > 0 || st.sh == 0)) {
    // a round inside the row: nothing to mask
#pragma unroll
    for (int i = 0; i < S; ++i) lm = fmaxf(lm, a.x[i]);
  } else {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int j = round_slot_index<W, T, VEC>(round, i, wid, lane);
      a.x[i] = j < C && j >= st.sh ? a.x[i] : -INFINITY;
      lm = fmaxf(lm, a.x[i]);
    }
  }
  st.m = fmaxf(st.m, wave_max_f32(lm));
  st.t = fmaxf(st.t, bound_below_max(st.m));
  bool done = false;
  if (!st.ovf) {
    if (ballot(lm > st.t) == 0) {
      done = true;   // no candidate in this round (the common case)
    } else {
      int lc = 0;
#pragma unroll
      for (int i = 0; i < S; ++i) lc += a.x[i] > st.t ? 1 : 0;
      // per-lane counts and their prefix sum place each lane's entries: lane L appends its k-th
      // entry at n + (entries of lanes < L) + k, and an entry not appended is written to the
      // lane's trash slot (tr) instead, so the appends need no per-slot ballot or branch
      int incl = scan_i32(lc);
      int cnt = __builtin_amdgcn_readlane(incl, kWave - 1);
      // a list that still has its indices is tightened before it gives them up
      if (st.n + cnt > (st.noidx ? cap : icap)) {
        tighten<S>(bv, bi, st.n, st.t, a.x, st.m, st.noidx, lane);
        lc = 0;
#pragma unroll
        for (int i = 0; i < S; ++i) lc += a.x[i] > st.t ? 1 : 0;
        incl = scan_i32(lc);
        cnt = __builtin_amdgcn_readlane(incl, kWave - 1);
        if (st.n + cnt > cap) {
          // the list cannot hold every entry above the bound: keep its sum and go on summing
          st.ovf = true;
          st.tov = st.t;
          double s;
          int c;
          list_sum_count(bv, st.n, st.tov, lane, s, c);
          if (lane == 0) {
            st.acc_s += s;
            st.acc_c += c;
          }
        }
      }
      if (!st.ovf) {
        if (st.n + cnt > icap) st.noidx = true;
        int pos = st.n + incl - lc;
        // the bound again, as a value the compiler does not match with the count's compares: the
        // appends then compare into VCC rather than keep 16 lane masks in scalar registers
        const float tw = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(st.t)));
        if (ballot(lc > 1) == 0) {
          // a sparse round: no lane has more than one entry, which is then its maximum lm
          const bool p = lc == 1;
          *(p ? bv + pos : tr) = lm;
          if (!st.noidx) {
            int id = 0;
#pragma unroll
            for (int i = 0; i < S; ++i)
              id = a.x[i] == lm ? round_slot_index<W, T, VEC>(round, i, wid, lane) - st.sh : id;
            *(p ? bi + pos : reinterpret_cast<int*>(tr)) = id;
          }
        } else if (ballot(lc > 2) == 0) {
          // at most two entries per lane: its first and its last entry in slot order (the same
          // entry when it has one), so the list's order is that of the per-slot appends below
          // (2048 x 131072 at N(0, 0.001^2): most rounds after the first few dozen)
          auto pair = [&](auto idx) {
            constexpr bool IDX = decltype(idx)::value;
            float fv = 0.0f, lv = 0.0f;
            int fs = 0, ls = 0;
#pragma unroll
            for (int i = 0; i < S; ++i) {
              const bool p = a.x[i] > tw;
              lv = p ? a.x[i] : lv;
              if constexpr (IDX) ls = p ? i : ls;
            }
#pragma unroll
            for (int i = S - 1; i >= 0; --i) {
              const bool p = a.x[i] > tw;
              fv = p ? a.x[i] : fv;
              if constexpr (IDX) fs = p ? i : fs;
            }
            *(lc >= 1 ? bv + pos : tr) = fv;
            *(lc == 2 ? bv + pos + 1 : tr) = lv;
            if constexpr (IDX) {
              *(lc >= 1 ? bi + pos : reinterpret_cast<int*>(tr)) = round_slot_index<W, T, VEC>(round, fs, wid, lane) - st.sh;
              *(lc == 2 ? bi + pos + 1 : reinterpret_cast<int*>(tr)) =
                  round_slot_index<W, T, VEC>(round, ls, wid, lane) - st.sh;
            }
          };
          if (st.noidx) pair(std::false_type{});
          else pair(std::true_type{});
        } else if (st.noidx) {
#pragma unroll
          for (int i = 0; i < S; ++i) {
            const bool p = a.x[i] > tw;
            *(p ? bv + pos : tr) = a.x[i];
            pos += p ? 1 : 0;
          }
        } else {
#pragma unroll
          for (int i = 0; i < S; ++i) {
            const bool p = a.x[i] > tw;
            *(p ? bv + pos : tr) = a.x[i];
            *(p ? bi + pos : reinterpret_cast<int*>(tr)) = round_slot_index<W, T, VEC>(round, i, wid, lane) - st.sh;
            pos += p ? 1 : 0;
          }
        }
        st.n += cnt;
        done = true;
      }
    }
  }
  if (!done) {
    if (isnan(st.tov)) st.tov = st.t;   // forced overflow: the first round's bound
    // per-lane fp32 partial sum of the round (the bound derived from it allows for its rounding)
    float rs = 0.0f;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const bool k = a.x[i] > st.tov;
      rs += k ? a.x[i] : 0.0f;
      st.acc_c += k ? 1 : 0;
    }
    st.acc_s += (double)rs;
  }
}

// bytes of the resource of a streamed row (or window) of C elements: 128-bit rounds take whole
// dwords (the buffer range check is per dword), so a 16-bit window of odd length takes the dword
// that holds its last element (its other half is masked; a dword never crosses a page)
template <typename T, bool VEC>
__device__ __forceinline__ uint32_t stream_bytes(int C) {
  const uint32_t b = (uint32_t)(kElemBytes<T> * C);
  return VEC ? (b + 3u) & ~3u : b;
}

// the first round of a row (or stretch), loaded ahead of stream_span (C = 0: no row, no traffic)
template <int W, typename T, bool VEC>
__device__ __forceinline__ void stream_first(const void* __restrict__ row, int C, int lane, int wid, Round<T, VEC>& a) {
  load_round<W, T, VEC>(make_rsrc_u(row, stream_bytes<T, VEC>(C)), 0, wid, lane, a);
}

// Stream this wavefront's share of a row (or of a stretch of one: `row`, `out_row` and C narrowed
// to it) once: loads run one round ahead of the candidate scan, and every dense output element
// (gradient or mask; `out_row` null in candidate-list mode) gets its zero placeholder.  `a` holds
// the first round, from stream_first.  With st.sh > 0 (candidate-list mode only), `row` is the
// start of a window st.sh elements before the row and C the window's length.
template <int W, typename T, int MODE, bool VEC>
__device__ __forceinline__ void stream_span(const void* __restrict__ row, void* out_row, int C, int lane, int wid,
                                            float* bv, int* bi, float* tr, int cap, int icap,
                                            StreamState& st, Round<T, VEC>& a) {
  constexpr int per_round = kWave * W * Round<T, VEC>::kSlots;   // elements per round of the row
  const int rounds = (C + per_round - 1) / per_round;
  const uint32_t row_bytes = (uint32_t)(kElemBytes<T> * C);
  const rsrc_t in = make_rsrc_u(row, stream_bytes<T, VEC>(C));
  rsrc_t out = make_rsrc(nullptr, 0u);
  if constexpr (MODE == kGrad) out = make_rsrc_u(out_row, row_bytes);
  else if constexpr (MODE == kMask) out = make_rsrc_u(out_row, (uint32_t)C);
  Round<T, VEC> b;
  // stores to a zero-size resource (no traffic) so that the wait counts on entry match those of
  // the loop's back edge (a round's loads, then a round's stores)
  __builtin_amdgcn_sched_barrier(0);
  zero_round<W, T, MODE, VEC>(make_rsrc(nullptr, 0u), 0, wid, lane);
  __builtin_amdgcn_sched_barrier(0);
  int k = 0;
  while (true) {
    load_round<W, T, VEC>(k + 1 < rounds ? in : make_rsrc_u(row, 0u), k + 1, wid, lane, b);
    zero_round<W, T, MODE, VEC>(out, k, wid, lane);
    scan_round<W, T, VEC>(a, k, C, wid, lane, bv, bi, tr, cap, icap, st);
    if (++k >= rounds) break;
    load_round<W, T, VEC>(k + 1 < rounds ? in : make_rsrc_u(row, 0u), k + 1, wid, lane, a);
    zero_round<W, T, MODE, VEC>(out, k, wid, lane);
    scan_round<W, T, VEC>(b, k, C, wid, lane, bv, bi, tr, cap, icap, st);
    if (++k >= rounds) break;
  }
}

// The wavefront's contribution to the overflow solve's first lower bound: the sum and count of a
// set of its entries (the accumulated entries > tov after an overflow, else its list entries > t)
// and a bound on their magnitudes.  H of the union over wavefronts is <= tau.
__device__ __forceinline__ void stream_lower_set(const StreamState& st, const float* bv, int lane, double& s, int& c,
                                                 float& B) {
  if (st.ovf) {
    s = wave_sum_f64(st.acc_s);
    c = wave_sum_i32(st.acc_c);
    B = fmaxf(fabsf(st.m), fabsf(st.tov));
  } else {
    list_sum_count(bv, st.n, st.t, lane, s, c);
    B = fmaxf(fabsf(st.m), fabsf(st.t));
  }
  if (c == 0) B = 0.0f;
}

// The wavefronts' candidate lists of a row (or of a stretch of one) in `sh` hold every entry above
// each wavefront's final bound; cut them at the block maximum and resolve tau and kappa into
// sh.tau / sh.kappa (valid after the caller's next barrier).
// (SH = BlockSharedBig: the lists are padded (pad_list) and the fixed-point steps of a long merged
// list run on all four wavefronts, each summing its own list)
template <typename SH>
__device__ __forceinline__ void block_merge_resolve(SH& sh, int n, int wid, int lane) {
  constexpr bool kBig = std::is_same<SH, BlockSharedBig>::value;
  const float* bv = sh.bval[wid];
  const float M = fmaxf(fmaxf(sh.wmax[0], sh.wmax[1]), fmaxf(sh.wmax[2], sh.wmax[3]));
  const float tb = bound_below_max(M);
  int nb = 0;
  for (int p0 = 0; p0 < n; p0 += kWave) {
    const int p = p0 + lane;
    nb += __popcll(ballot(p < n && bv[p] > tb));
  }
  if (lane == 0) sh.wsel[wid] = nb;
  __syncthreads();
  const int ntot = (sh.wsel[0] + sh.wsel[1]) + (sh.wsel[2] + sh.wsel[3]);
  if (ntot > 0 && ntot <= kWave) {
    int off = 0;
    for (int w = 0; w < wid; ++w) off += sh.wsel[w];
    for (int p0 = 0; p0 < n; p0 += kWave) {
      const int p = p0 + lane;
      const float v = p < n ? bv[p] : -INFINITY;
      const bool k = v > tb;
      const uint64_t b = ballot(k);
      if (k) sh.sel[off + rank_in(b)] = v;
      off += __popcll(b);
    }
    __syncthreads();
    if (wid == 0) {
      const float c = lane < ntot ? sh.sel[lane] : -INFINITY;
      const double tt = clamp_below_max(select_small(c, ntot, lane), M);
      const int kk = __popcll(ballot(lane < ntot && c > rd32(tt)));
      if (lane == 0) {
        sh.tau = tt;
        sh.kappa = kk;
      }
    }
  } else if (ntot > kWave && kBig) {
    // fixed-point iterations over the four lists, each wavefront summing its own, the partials
    // added in a fixed order (every wavefront takes the same steps)
    auto all_sum_count = [&](float thr, double& s, int& c) {
      double sw;
      int cw;
      list4_sum_count(sh.bval[wid], n, thr, lane, sw, cw);
      __syncthreads();
      if (lane == 0) {
        sh.red_s[wid] = sw;
        sh.red_c[wid] = cw;
      }
      __syncthreads();
      s = (sh.red_s[0] + sh.red_s[1]) + (sh.red_s[2] + sh.red_s[3]);
      c = (sh.red_c[0] + sh.red_c[1]) + (sh.red_c[2] + sh.red_c[3]);
    };
    double tt = (double)tb, s;
    int c;
    all_sum_count(tb, s, c);
    double res_t = NAN;
    int res_k = 0;
    for (int it = 0; it <= ntot + 1; ++it) {
      const double tn = (s - 1.0) / (double)c;
      double s2;
      int c2;
      all_sum_count(rd32(tn), s2, c2);
      if (c2 == c || !(tn > tt)) {
        res_t = tn;
        res_k = c2;
        break;
      }
      tt = tn;
      s = s2;
      c = c2;
    }
    const double tc = clamp_below_max(res_t, M);
    if (tc != res_t) {
      double s3;
      res_t = tc;
      all_sum_count(rd32(res_t), s3, res_k);
    }
    if (threadIdx.x == 0) {
      sh.tau = res_t;
      sh.kappa = res_k;
    }
  } else if (ntot > kWave) {
    if (wid == 0) {
      // fixed-point iterations over the four lists (wavefront 0)
      auto all_sum_count = [&](float thr, double& s, int& c) {
        double st = 0.0;
        int ct = 0;
        for (int w = 0; w < kWavesPerBlock; ++w) {
          double sw;
          int cw;
          list_sum_count(sh.bval[w], sh.wn[w], thr, lane, sw, cw);
          st += sw;
          ct += cw;
        }
        s = st;
        c = ct;
      };
      double tt = (double)tb, s;
      int c;
      all_sum_count(tb, s, c);
      double res_t = NAN;
      int res_k = 0;
      for (int it = 0; it <= ntot + 1; ++it) {
        const double tn = (s - 1.0) / (double)c;
        double s2;
        int c2;
        all_sum_count(rd32(tn), s2, c2);
        if (c2 == c || !(tn > tt)) {
          res_t = tn;
          res_k = c2;
          break;
        }
        tt = tn;
        s = s2;
        c = c2;
      }
      const double tc = clamp_below_max(res_t, M);
      if (tc != res_t) {
        double s3;
        res_t = tc;
        all_sum_count(rd32(res_t), s3, res_k);
      }
      if (lane == 0) {
        sh.tau = res_t;
        sh.kappa = res_k;
      }
    }
  } else if (threadIdx.x == 0) {
    sh.tau = NAN;
    sh.kappa = 0;
  }
}

// ------------------------------------------------------------------------------------------------
// The overflow solve: tau of a row whose candidates did not fit the LDS lists, from the row in
// memory, in a bounded number of passes, by W wavefronts (W = 1: the calling wavefront alone;
// W = kWavesPerBlock: every thread of the block calls).
//
//   1. A histogram pass: count and fp64 sum of the entries in (t1, M] (t1 a lower bound on tau, M
//      the row maximum) in bins of width w = 2^e, bin b holding t1 + b*w <= z < t1 + (b+1)*w
//      (bins and edges exact in fp64; LDS atomics).  G(e) = sum_{z >= e} (z - e) is decreasing
//      and G(tau) = 1, so the highest bin whose lower edge has G >= 1 holds tau.
//   2. When that bin holds more entries than the LDS list, another histogram pass splits it by the
//      order-preserving keys of its floats (at most 4 such passes: each divides a key range of
//      at most 2^32 by the number of bins; a bin of one key holds equal values, none of which is
//      in the support since tau >= the bin's edge).
//   3. A collect pass gathers the bin's entries into the LDS list and sums every entry above the
//      bin exactly (fixed order, fp64); the support is those entries plus the top j of the bin,
//      with j from the sparsemax condition k z_(k) > S_k - 1 (a sort of <= 64 entries, or
//      fixed-point steps over the list); the result is checked to lie in the bin.
//   4. The histogram's sums are fp64 atomics, so a bin choice can be off when G is within a few
//      ulps of 1; the check in 3 catches that, and a bisection over the keys of [t1, M] with exact
//      fixed-order G (at most 34 passes) gives the answer then.
// Every decision that fixes the result is taken on fixed-order fp64 sums, so the result does not
// depend on the order of the atomics.

struct SelMem {
  unsigned* hcnt;
  double* hsum;
  float* list;
  int nbins;    // bins per histogram pass: a multiple of 64
  int cap;      // list capacity of the collect pass
  double* red_s;
  int* red_c;
  int* ncol;
};

// the histogram, the list and the block scalars share LDS bytes under different types: every
// change of role goes through this barrier (a fence keeps the compiler from moving the LDS
// accesses across it)
template <int W>
__device__ __forceinline__ void sel_sync() {
  if constexpr (W == 1) {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  } else {
    __syncthreads();
  }
}

// fp64 sum and count over the W wavefronts in a fixed order (every lane receives them)
template <int W>
__device__ __forceinline__ void sel_reduce(double& s, int& c, const SelMem& sm, int wid, int lane) {
  s = wave_sum_f64(s);
  c = wave_sum_i32(c);
  if constexpr (W > 1) {
    static_assert(W == kWavesPerBlock, "one wavefront or the whole block");
    __syncthreads();
    if (lane == 0) {
      sm.red_s[wid] = s;
      sm.red_c[wid] = c;
    }
    __syncthreads();
    s = (sm.red_s[0] + sm.red_s[1]) + (sm.red_s[2] + sm.red_s[3]);
    c = (sm.red_c[0] + sm.red_c[1]) + (sm.red_c[2] + sm.red_c[3]);
    __syncthreads();
  }
}

// One pass over a row: f(z, j) for every slot of every round (z = -inf for slots past the row;
// all lanes call f for a slot together), W wavefronts interleaved as in the streaming rounds.  DB:
// two rounds of loads in flight (fwl_overflow_rows); without it one round at a time, so that the
// solve inside the streaming kernels (no workspace) holds no more registers than their stream.
template <int W, typename T, bool VEC, bool DB, typename F>
__device__ __forceinline__ void row_pass(const void* row, int C, int lane, int wid, F&& f) {
  constexpr int S = Round<T, VEC>::kSlots;
  constexpr int per_round = kWave * W * S;
  const int rounds = (C + per_round - 1) / per_round;
  const rsrc_t in = make_rsrc_u(row, stream_bytes<T, VEC>(C));
  const rsrc_t none = make_rsrc_u(row, 0u);
  auto process = [&](Round<T, VEC>& a, int k) {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int j = round_slot_index<W, T, VEC>(k, i, wid, lane);
      f(j < C ? a.x[i] : -INFINITY, j);
    }
  };
  if constexpr (DB) {
    Round<T, VEC> a, b;
    load_round<W, T, VEC>(in, 0, wid, lane, a);
    for (int k = 0; k < rounds; k += 2) {
      load_round<W, T, VEC>(k + 1 < rounds ? in : none, k + 1, wid, lane, b);
      process(a, k);
      if (k + 1 >= rounds) break;
      load_round<W, T, VEC>(k + 2 < rounds ? in : none, k + 2, wid, lane, a);
      process(b, k + 1);
    }
  } else {
    for (int k = 0; k < rounds; ++k) {
      Round<T, VEC> a;
      load_round<W, T, VEC>(in, k, wid, lane, a);
      process(a, k);
    }
  }
}

// Bins of one histogram pass.  Linear: bin b holds base + b*w <= z < base + (b+1)*w for z > lo
// (w a power of two: the edges are exact in fp64); by key: bin b holds the floats whose keys lie
// in [kbase + (b << sh), kbase + ((b + 1) << sh)), for keys in [kbase, kmax].
struct BinMap {
  bool by_key;
  double base, w, inv_w;
  float lo;
  int kbase, kmax, sh;
  int nb;
};

__device__ __forceinline__ int canon_key(float z) { return fkey(z + 0.0f); }   // -0.0 -> +0.0

__device__ __forceinline__ double bin_edge(const BinMap& bm, int b) {
  if (bm.by_key) return (double)fkey_inv((int)((int64_t)bm.kbase + ((int64_t)b << bm.sh)));
  return bm.base + (double)b * bm.w;
}

// bin of z, or -1 outside the map's range
__device__ __forceinline__ int bin_of(const BinMap& bm, float z) {
  if (bm.by_key) {
    const int k = canon_key(z);
    if (!(z == z) || k < bm.kbase || k > bm.kmax) return -1;
    return (int)(((int64_t)k - bm.kbase) >> bm.sh);
  }
  if (!(z > bm.lo) || !(z < INFINITY)) return -1;
  const double d = ((double)z - bm.base) * bm.inv_w;
  int b = d < (double)bm.nb ? (int)d : bm.nb - 1;
  b = b < 0 ? 0 : b;
  // the difference may round when z and the base are far apart: place z by exact compares
  if ((double)z < bin_edge(bm, b)) b = b > 0 ? b - 1 : 0;
  else if (b + 1 < bm.nb && (double)z >= bin_edge(bm, b + 1)) b += 1;
  return b;
}

// linear bins over (t1, M]: the smallest power-of-two width with nbins * w >= M - t1
__device__ __forceinline__ BinMap linear_bins(float t1, float M, int nbins) {
  BinMap bm;
  bm.by_key = false;
  bm.base = (double)t1;
  bm.lo = t1;
  int e = 0;
  const double span = ((double)M - (double)t1) / (double)nbins;
  frexp(span > 0.0 ? span : 0x1p-1074, &e);   // span < 2^e
  bm.w = ldexp(1.0, e);
  bm.inv_w = ldexp(1.0, -e);
  bm.kbase = bm.kmax = bm.sh = 0;
  bm.nb = nbins;
  return bm;
}

// key bins over the floats in [lo, hi) (lo, hi exact fp64 values, lo < hi)
__device__ __forceinline__ BinMap key_bins(double lo, double hi, int nbins) {
  float f = (float)lo;
  if ((double)f < lo) f = next_f32(f);
  float g = (float)hi;
  if ((double)g >= hi) g = prev_f32(g);
  BinMap bm;
  bm.by_key = true;
  bm.base = bm.w = bm.inv_w = 0.0;
  bm.lo = f;
  bm.kbase = canon_key(f);
  bm.kmax = canon_key(g);
  if (bm.kmax < bm.kbase) bm.kmax = bm.kbase;
  const int64_t range = (int64_t)bm.kmax - bm.kbase + 1;
  int sh = 0;
  while (((range - 1) >> sh) >= nbins) ++sh;
  bm.sh = sh;
  bm.nb = (int)(((range - 1) >> sh) + 1);
  return bm;
}

// one histogram pass (counts exact, sums approximate: fp64 atomics in any order)
template <int W, typename T, bool VEC>
__device__ void hist_pass(const void* row, int C, const BinMap& bm, const SelMem& sm, int lane, int wid) {
  const int t0 = W > 1 ? (int)threadIdx.x : lane;
  for (int b = t0; b < sm.nbins; b += kWave * W) {
    sm.hcnt[b] = 0u;
    sm.hsum[b] = 0.0;
  }
  sel_sync<W>();
  row_pass<W, T, VEC, true>(row, C, lane, wid, [&](float z, int) {
    const int b = bin_of(bm, z);
    if (b >= 0) {
      __hip_atomic_fetch_add(sm.hcnt + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_fetch_add(sm.hsum + b, (double)z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  });
  sel_sync<W>();
}

// The highest bin whose lower edge e has G(e) = S_up + sum_{bins >= b} - (C_up + count_{bins >= b}) e
// >= 1, by one wavefront (every lane gets the results): lane l holds bins nbins-1 - (l*q + i),
// i < q, so an inclusive scan over the lanes adds the bins from the top.  Returns the bin, its
// count and the approximate count and sum of the entries above it.
__device__ int find_boundary(const BinMap& bm, const SelMem& sm, int C_up, double S_up, int lane, int& cnt_b,
                             int& c_above, double& s_above) {
  const int q = sm.nbins / kWave;
  int tc = 0;
  double ts = 0.0;
  for (int i = 0; i < q; ++i) {
    const int b = sm.nbins - 1 - (lane * q + i);
    tc += (int)sm.hcnt[b];
    ts += sm.hsum[b];
  }
  int tot;
  const int pc = wave_excl_scan_i32(tc, tot);   // exclusive: the lanes above this one
  const double ps_incl = scan_f64<kWave>(ts);
  const double ps = ps_incl - ts;
  const double tsum = readlane_f64(ps_incl, kWave - 1);
  int ac = C_up + pc;
  double as = S_up + ps;
  int found = -1, f_cnt = 0, f_ac = 0;
  double f_as = 0.0;
  for (int i = 0; i < q; ++i) {
    const int b = sm.nbins - 1 - (lane * q + i);
    const int cb = (int)sm.hcnt[b];
    const double sb = sm.hsum[b];
    const int a2 = ac + cb;
    const double s2 = as + sb;
    if (found < 0 && b < bm.nb && s2 - (double)a2 * bin_edge(bm, b) >= 1.0) {
      found = b;
      f_cnt = cb;
      f_ac = ac;
      f_as = as;
    }
    ac = a2;
    as = s2;
  }
  const uint64_t has = ballot(found >= 0);
  if (has == 0) {
    // no edge with G >= 1 (only from rounding: G(t1) >= 1): the lowest bin
    cnt_b = (int)sm.hcnt[0];
    c_above = C_up + tot - cnt_b;
    s_above = S_up + tsum - sm.hsum[0];
    return 0;
  }
  const int src = (int)__builtin_ctzll(has);   // the lowest lane: the highest bin
  cnt_b = __builtin_amdgcn_readlane(f_cnt, src);
  c_above = __builtin_amdgcn_readlane(f_ac, src);
  s_above = readlane_f64(f_as, src);
  return __builtin_amdgcn_readlane(found, src);
}

// tau of the support {entries above the bin} U {the top j of the bin's n entries in the list},
// given the exact count and sum above the bin (C_hi, S_hi); the bin's entries are >= lo and < hi.
// Returns false if tau does not lie in [lo, hi) (then the bin was not the boundary).
__device__ bool resolve_bin(const float* list, int n, int C_hi, double S_hi, double lo, double hi, int lane,
                            double& tau, int& kappa) {
  int j = 0;
  double Sj = 0.0;
  if (n <= kWave) {
    const float c = lane < n ? list[lane] : -INFINITY;
    int key = canon_key(lane < n ? c : -INFINITY);
    key = sort_desc_i<kWave>(key, lane);
    const float v = fkey_inv(key);
    const double P = scan_f64<kWave>(lane < n ? (double)v : 0.0);
    const uint64_t in = ballot(lane < n && (double)v * (double)(C_hi + lane + 1) > S_hi + P - 1.0);
    j = in == 0 ? 0 : 64 - (int)__builtin_clzll(in);
    j = uniform(j);
    Sj = j > 0 ? readlane_f64(P, j - 1) : 0.0;
  } else {
    // fixed-point steps from lo (a lower bound on tau if the bin is the boundary)
    double t = lo, s = 0.0;
    int c = 0, it = 0;
    list_sum_count(list, n, rd32(t), lane, s, c);
    for (; it < n + 2; ++it) {
      if (C_hi + c == 0) break;
      const double tn = (S_hi + s - 1.0) / (double)(C_hi + c);
      double s2;
      int c2;
      list_sum_count(list, n, rd32(tn), lane, s2, c2);
      if (c2 == c || !(tn > t)) {
        s = s2;
        c = c2;
        break;
      }
      t = tn;
      s = s2;
      c = c2;
    }
    j = c;
    Sj = s;
  }
  kappa = C_hi + j;
  if (kappa == 0) return false;
  tau = (S_hi + Sj - 1.0) / (double)kappa;
  return tau >= lo && tau < hi;
}

// exact fixed-order G(v) = sum_{z > v} (z - v) of the row, as (sum, count) of the entries > v
template <int W, typename T, bool VEC, bool DB>
__device__ void row_above(const void* row, int C, float v, const SelMem& sm, int lane, int wid, double& s, int& c) {
  double acc = 0.0;
  int cnt = 0;
  row_pass<W, T, VEC, DB>(row, C, lane, wid, [&](float z, int) {
    const bool k = z > v;
    acc += k ? (double)z : 0.0;
    cnt += k ? 1 : 0;
  });
  s = acc;
  c = cnt;
  sel_reduce<W>(s, c, sm, wid, lane);
}

// tau < M: only when the 1 of S - 1 was lost (|z| >= 2^53) is it clamped below the maximum, and
// kappa counted again
template <int W, typename T, bool VEC, bool DB>
__device__ void clamp_row(const void* row, int C, float M, const SelMem& sm, int lane, int wid, double& tau,
                          int& kappa) {
  const double tc = clamp_below_max(tau, M);
  if (tc != tau) {
    double s;
    int c;
    tau = tc;
    row_above<W, T, VEC, DB>(row, C, rd32(tau), sm, lane, wid, s, c);
    kappa = c;
  }
}

// Bisection over the keys of [t1, M] with exact fixed-order G at every step (at most 32 passes
// over the row, then one for the sums): G(a) >= 1 > G(b) brackets tau in [a, b) for adjacent keys
// a, b, so the support is {z > a}.  Needs nothing but the row; the last resort of
// select_in_memory and the whole solve where there is no workspace to defer rows to.
template <int W, typename T, bool VEC, bool DB>
__device__ void select_bisect(const void* row, int C, float t1, float M, const SelMem& sm, int lane, int wid,
                              double& tau, int& kappa) {
  tau = NAN;
  kappa = 0;
  if (!isfinite(M) || !(t1 < M)) return;
  int ka = canon_key(t1), kb = canon_key(M);
  while ((int64_t)kb - ka > 1) {
    const int km = (int)(((int64_t)ka + kb) >> 1);
    const float v = fkey_inv(km);
    double s;
    int c;
    row_above<W, T, VEC, DB>(row, C, v, sm, lane, wid, s, c);
    if (s - (double)c * (double)v >= 1.0) ka = km;
    else kb = km;
  }
  double s;
  int c;
  row_above<W, T, VEC, DB>(row, C, fkey_inv(ka), sm, lane, wid, s, c);
  kappa = c;
  tau = c > 0 ? (s - 1.0) / (double)c : NAN;
  clamp_row<W, T, VEC, DB>(row, C, M, sm, lane, wid, tau, kappa);
}

template <int W, typename T, bool VEC>
__device__ void select_in_memory(const void* row, int C, float t1, float M, const SelMem& sm, int lane, int wid,
                                 double& tau, int& kappa) {
  tau = NAN;
  kappa = 0;
  if (!isfinite(M) || !(t1 < M)) return;   // no finite maximum: no finite tau (as the list path)
  BinMap bm = linear_bins(t1, M, sm.nbins);
  int C_up = 0;
  double S_up = 0.0;
  bool done = false;
  for (int pass = 0; pass < 6 && !done; ++pass) {
    hist_pass<W, T, VEC>(row, C, bm, sm, lane, wid);
    int bstar = 0, cnt_b = 0, c_above = 0;
    double s_above = 0.0;
    if (W == 1 || wid == 0) bstar = find_boundary(bm, sm, C_up, S_up, lane, cnt_b, c_above, s_above);
    if constexpr (W > 1) {
      if (threadIdx.x == 0) {
        sm.red_c[0] = bstar;
        sm.red_c[1] = cnt_b;
        sm.red_c[2] = c_above;
        sm.red_s[0] = s_above;
      }
      __syncthreads();
      bstar = sm.red_c[0];
      cnt_b = sm.red_c[1];
      c_above = sm.red_c[2];
      s_above = sm.red_s[0];
      __syncthreads();
    }
    const double lo = bin_edge(bm, bstar);
    const double hi = bstar + 1 < bm.nb ? bin_edge(bm, bstar + 1)
                                        : (bm.by_key ? (double)next_f32(fkey_inv(bm.kmax)) : bm.base + bm.nb * bm.w);
    sel_sync<W>();
    const bool single = bm.by_key && bm.sh == 0;   // one key per bin: equal values, none in the support
    if (cnt_b > sm.cap && !single && pass < 5) {
      bm = key_bins(lo, hi, sm.nbins);
      C_up = c_above;
      S_up = s_above;
      continue;
    }
    // collect pass: the bin's entries into the list, exact count and sum above the bin
    if constexpr (W > 1) {
      if (threadIdx.x == 0) *sm.ncol = 0;
      __syncthreads();
    }
    int ncol = 0;
    bool lost = false;
    double acc = 0.0;
    int cnt = 0;
    row_pass<W, T, VEC, true>(row, C, lane, wid, [&](float z, int) {
      const double zd = (double)z;
      const bool above = zd >= hi;
      acc += above ? zd : 0.0;
      cnt += above ? 1 : 0;
      const bool in = !single && zd >= lo && zd < hi;
      const uint64_t bl = ballot(in);
      if (bl != 0) {
        const int k = __popcll(bl);
        int base;
        if constexpr (W > 1) {
          int b0 = 0;
          if (lane == 0) b0 = atomicAdd(sm.ncol, k);
          base = __builtin_amdgcn_readfirstlane(b0);
        } else {
          base = ncol;
          ncol += k;
        }
        const int pos = base + rank_in(bl);
        if (in && pos < sm.cap) sm.list[pos] = z;
        if (base + k > sm.cap) lost = true;
      }
    });
    double S_hi = acc;
    int C_hi = cnt;
    sel_reduce<W>(S_hi, C_hi, sm, wid, lane);
    if constexpr (W > 1) {
      ncol = *sm.ncol;
      const int lost_any = __syncthreads_or(lost ? 1 : 0);
      lost = lost_any != 0;
    }
    sel_sync<W>();
    if (!lost) {
      bool ok = false;
      double tt = NAN;
      int kk = 0;
      if (W == 1 || wid == 0) ok = resolve_bin(sm.list, ncol, C_hi, S_hi, lo, hi, lane, tt, kk);
      if constexpr (W > 1) {
        if (threadIdx.x == 0) {
          sm.red_c[0] = ok ? 1 : 0;
          sm.red_c[1] = kk;
          sm.red_s[0] = tt;
        }
        __syncthreads();
        ok = sm.red_c[0] != 0;
        kk = sm.red_c[1];
        tt = sm.red_s[0];
        __syncthreads();
      }
      if (ok) {
        tau = tt;
        kappa = kk;
        done = true;
      }
    }
    break;
  }
  if (!done) select_bisect<W, T, VEC, true>(row, C, t1, M, sm, lane, wid, tau, kappa);
  else clamp_row<W, T, VEC, true>(row, C, M, sm, lane, wid, tau, kappa);
}

// The support of a row solved in memory, written from the row: the gradient (inv) or mask (1) at
// every entry > Hf but the label (the placeholders hold 0 everywhere else), or the candidate list
// (at most o.ccap entries, in pass order).
template <int W, typename T, int MODE, bool VEC, bool DB>
__device__ void write_support(const void* row, int64_t r, int C, int yr, float Hf, float inv, const Outs& o,
                              int* wsel, int lane, int wid) {
  if constexpr (MODE == kGrad || MODE == kMask) {
    row_pass<W, T, VEC, DB>(row, C, lane, wid, [&](float z, int j) {
      if (z > Hf && j != yr) {
        if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + j, inv);
        else o.mask[r * (int64_t)C + j] = 1;
      }
    });
  } else {
    // candidate lists in a deterministic order: per round, the wavefronts in order, then their slots
    constexpr int S = Round<T, VEC>::kSlots;
    constexpr int per_round = kWave * W * S;
    const int rounds = (C + per_round - 1) / per_round;
    const rsrc_t in = make_rsrc_u(row, (uint32_t)(kElemBytes<T> * C));
    float* cv = o.cval != nullptr ? o.cval + r * (int64_t)o.cstride : nullptr;   // null: indices only
    int32_t* ci = o.cidx + r * (int64_t)o.cstride;
    int base = 0;
    for (int k = 0; k < rounds; ++k) {
      Round<T, VEC> a;
      load_round<W, T, VEC>(in, k, wid, lane, a);
      int mine = 0;
#pragma unroll
      for (int i = 0; i < S; ++i) {
        const int j = round_slot_index<W, T, VEC>(k, i, wid, lane);
        mine += __popcll(ballot(j < C && a.x[i] > Hf));
      }
      int off = base;
      if constexpr (W > 1) {
        __syncthreads();
        if (lane == 0) wsel[wid] = mine;
        __syncthreads();
        for (int w = 0; w < wid; ++w) off += wsel[w];
        base += (wsel[0] + wsel[1]) + (wsel[2] + wsel[3]);
      } else {
        base += mine;
      }
#pragma unroll
      for (int i = 0; i < S; ++i) {
        const int j = round_slot_index<W, T, VEC>(k, i, wid, lane);
        const bool sel = j < C && a.x[i] > Hf;
        const uint64_t b = ballot(sel);
        const int pos = off + rank_in(b);
        if (sel && pos < o.ccap) {
          if (cv != nullptr) cv[pos] = a.x[i];
          ci[pos] = j;
        }
        off += __popcll(b);
      }
    }
  }
}

// 16-bit rows of odd start in candidate-list mode (the two-pass op's read pass) stream a window
// from the 4-byte boundary below the row, one element longer (every dword of the 128-bit loads
// then lies in the window; the element in front of the row is masked): win_shift is that element
// count (0 or 1), 0 for every other row.  Nothing is stored through the window.
template <typename T, int MODE, bool V4>
__device__ __forceinline__ int win_shift(const void* row) {
  if constexpr (MODE == kCand && V4 && kElemBytes<T> == 2) return (int)((reinterpret_cast<uintptr_t>(row) >> 1) & 1);
  else return 0;
}

// (BIG: the long lists of BlockSharedBig, in candidate-list mode; a row one of whose wavefronts'
// lists outgrew its indices has its support, where the caller wants it listed, written from one
// more pass over the row)
template <typename T, int MODE, bool V4, bool BIG = false>
__global__ __launch_bounds__(kBlock) void fwl_block_rows(const void* __restrict__ z,
                                                         const int64_t* __restrict__ tgt, int64_t N,
                                                         int C, Outs o) {
  static_assert(!BIG || MODE == kCand, "long block lists: candidate-list mode only");
  using SH = std::conditional_t<BIG, BlockSharedBig, BlockShared>;
  __shared__ SH sh;
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  double bsum = 0.0;
  auto row_at = [&](int64_t rr) { return static_cast<const char*>(z) + rr * o.ld * kElemBytes<T>; };
  // the first round of the next row is loaded before this row is resolved, so that the stream of
  // every row after the first starts with its loads in flight
  Round<T, V4> first;
  auto first_round = [&](const void* p) {
    const int ws = win_shift<T, MODE, V4>(p);
    stream_first<kWavesPerBlock, T, V4>(static_cast<const char*>(p) - kElemBytes<T> * ws, C + ws, lane, wid, first);
  };
  if (blockIdx.x < N) first_round(row_at(blockIdx.x));
  const SelMem sm = {nullptr, nullptr, nullptr, 0, 0, sh.red_s, sh.red_c, nullptr};
  for (int64_t r = blockIdx.x; r < N; r += gridDim.x) {
    const void* row = row_at(r);
    const int64_t y64 = tgt[r];
    const bool yok = y64 >= 0 && y64 < C;
    const int yr = yok ? (int)y64 : -1;
    float* bv = sh.bval[wid];
    int* bi;
    if constexpr (BIG) bi = reinterpret_cast<int*>(sh.bval[wid] + (kWaveVCap - kCapMax));
    else bi = sh.bidx[wid];
    const int vcap = BIG && o.cap >= kCapMax ? kWaveVCap : o.cap;

    StreamState st = stream_state(o.force_generic != 0);
    st.sh = win_shift<T, MODE, V4>(row);
    void* out_row = nullptr;
    if constexpr (MODE == kGrad) out_row = static_cast<char*>(o.grad) + r * (int64_t)C * kElemBytes<T>;
    else if constexpr (MODE == kMask) out_row = o.mask + r * (int64_t)C;
    stream_span<kWavesPerBlock, T, MODE, V4>(static_cast<const char*>(row) - kElemBytes<T> * st.sh, out_row, C + st.sh,
                                             lane, wid, bv, bi, sh.trash[wid] + lane, vcap, o.cap, st, first);
    if constexpr (BIG) pad_list(bv, st.n, lane);
    if (lane == 0) {
      sh.wmax[wid] = st.m;
      sh.wn[wid] = st.n;
      sh.ovf[wid] = st.ovf;
      if constexpr (BIG) sh.wnx[wid] = st.noidx;
    }
    const int64_t rn = r + gridDim.x;
    if constexpr (MODE == kGrad || MODE == kMask) {
      // every wavefront's zero placeholders have landed before any support entry is rewritten
      wait_vmem();
    }
    if (rn < N) first_round(row_at(rn));
    __syncthreads();
    const bool overflow = sh.ovf[0] | sh.ovf[1] | sh.ovf[2] | sh.ovf[3];

    double tau = NAN;
    int kappa = 0;
    bool deferred = false;
    bool unlisted = false;   // candidate-list mode: support left unlisted (mark_unlisted)
    if (!overflow) {
      block_merge_resolve(sh, st.n, wid, lane);
      __syncthreads();
      tau = sh.tau;
      kappa = sh.kappa;
      const float Hf = rd32(tau);
      const float inv = (float)(o.scale / (double)kappa);
      if constexpr (MODE == kGrad || MODE == kMask) {
        // the zero placeholders stand for every other entry
        for (int p = lane; p < st.n; p += kWave) {
          const int id = bi[p];
          if (id == yr || !(bv[p] > Hf)) continue;
          if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + id, inv);
          else o.mask[r * (int64_t)C + id] = 1;
        }
      } else if (BIG && (sh.wnx[0] | sh.wnx[1] | sh.wnx[2] | sh.wnx[3])) {
        // some list kept values only: the support from the row, where it is listed at all
        unlisted = o.mark_unlisted != 0;
        if (kappa <= o.ccap && !unlisted)
          write_support<kWavesPerBlock, T, MODE, V4, true>(row, r, C, yr, Hf, inv, o, sh.wsel, lane, wid);
      } else {
        int ns = 0;
        for (int p0 = 0; p0 < st.n; p0 += kWave) {
          const int p = p0 + lane;
          ns += __popcll(ballot(p < st.n && bv[p] > Hf));
        }
        __syncthreads();
        if (lane == 0) sh.wsel[wid] = ns;
        __syncthreads();
        int off = 0;
        for (int w = 0; w < wid; ++w) off += sh.wsel[w];
        float* cv = o.cval != nullptr ? o.cval + r * (int64_t)o.cstride : nullptr;
        int32_t* ci = o.cidx + r * (int64_t)o.cstride;
        for (int p0 = 0; p0 < st.n; p0 += kWave) {
          const int p = p0 + lane;
          const float v = p < st.n ? bv[p] : -INFINITY;
          const bool k = v > Hf;
          const uint64_t b = ballot(k);
          if (k && off + rank_in(b) < o.ccap) {
            const int pos = off + rank_in(b);
            if (cv != nullptr) cv[pos] = v;
            ci[pos] = bi[p];
          }
          off += __popcll(b);
        }
      }
    } else {
      // the overflow solve, from the best lower bound the stream left: every wavefront's bound and
      // H of the union of the sets they summed
      double ls;
      int lc;
      float lB;
      stream_lower_set(st, bv, lane, ls, lc, lB);
      if (lane == 0) {
        sh.wlo[wid] = st.t;
        sh.wB[wid] = lB;
        sh.red_s[wid] = ls;
        sh.red_c[wid] = lc;
      }
      __syncthreads();
      const float M = fmaxf(fmaxf(sh.wmax[0], sh.wmax[1]), fmaxf(sh.wmax[2], sh.wmax[3]));
      const double S = (sh.red_s[0] + sh.red_s[1]) + (sh.red_s[2] + sh.red_s[3]);
      const int Cn = (sh.red_c[0] + sh.red_c[1]) + (sh.red_c[2] + sh.red_c[3]);
      const float B = fmaxf(fmaxf(sh.wB[0], sh.wB[1]), fmaxf(sh.wB[2], sh.wB[3]));
      float t1 = fmaxf(fmaxf(fmaxf(sh.wlo[0], sh.wlo[1]), fmaxf(sh.wlo[2], sh.wlo[3])), bound_below_max(M));
      t1 = fmaxf(t1, safe_lower32(S, Cn, B));
      __syncthreads();
      if (o.ovf_lo != nullptr) {
        // fwl_overflow_rows solves the row and writes its outputs
        deferred = true;
        if (threadIdx.x == 0) {
          o.ovf_lo[r] = t1;
          o.ovf_mx[r] = M;
        }
      } else {
        select_bisect<kWavesPerBlock, T, V4, false>(row, C, t1, M, sm, lane, wid, tau, kappa);
        __syncthreads();
        write_support<kWavesPerBlock, T, MODE, V4, false>(row, r, C, yr, rd32(tau), (float)(o.scale / (double)kappa), o,
                                                          sh.wsel, lane, wid);
      }
    }
    if (threadIdx.x == 0 && !overflow && o.ovf_lo != nullptr) o.ovf_lo[r] = NAN;

    if (threadIdx.x == 0 && !deferred) {
      const float Hf = rd32(tau);
      const float inv = (float)(o.scale / (double)kappa);
      const float zy = yok ? load_elem<T>(row, yr) : NAN;
      if (yok) {
        if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + yr, (zy > Hf ? inv : 0.0f) - o.scale_f);
        else if constexpr (MODE == kMask) o.mask[r * (int64_t)C + yr] = (uint8_t)(zy > Hf);
      }
      const double l64 = (1.0 - (double)zy) + tau;
      const float loss = (float)l64;
      if (o.H) o.H[r] = Hf;
      if (o.loss) o.loss[r] = loss;
      if (o.loss64) o.loss64[r] = l64;
      if (o.kappa) o.kappa[r] = kappa;
      if constexpr (MODE == kCand) o.ccnt[r] = unlisted ? -kappa : kappa;
      bsum += (double)loss;
    }
    __syncthreads();
  }
  mean_epilogue(bsum, o);
}

// ------------------------------------------------------------------------------------------------
// fwl_wave_stream_rows: one wavefront per row for mid-range C.  The row is streamed once (loads
// one round ahead, zero placeholders for every output), its candidates kept in the wavefront's
// LDS list, which is then cut at the final bound max - 1 and resolved like a register row; only
// the support entries and the label are rewritten.  No block-wide barrier: each wavefront runs
// its own rows, as in fwl_wave_rows.  A row whose list overflows is solved in memory by its
// wavefront (select_in_memory with W = 1).
template <typename T, int MODE, bool V4, bool LONG>
__global__ __launch_bounds__(kBlock) void fwl_wave_stream_rows(const void* __restrict__ z,
                                                               const int64_t* __restrict__ tgt, int64_t N,
                                                               int C, Outs o) {
  constexpr int kVCap = LONG ? kStreamVCapLong : kWaveVCap;   // (LONG: the two-pass op's read pass)
  __shared__ WaveShared<kVCap> s_w[kWavesPerBlock];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  const int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wid;   // this wavefront's rows: w + k*stride
  const int nrows = w < N ? (int)((N - 1 - w) / stride + 1) : 0;   // <= kRowsPerWave (host grid)
  float* bv = s_w[wid].val;
  int* bi = reinterpret_cast<int*>(s_w[wid].val + (kVCap - kCapMax));
  const SelMem sm = {nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr};
  // the default capacity takes the whole value list; a smaller one (fwl_options) shrinks both
  const int vcap = o.cap >= kCapMax ? kVCap : o.cap;
  const int icap = o.cap < kCapMax ? o.cap : kCapMax;
  const int64_t my_y = lane < nrows ? tgt[w + (int64_t)lane * stride] : 0;
  float my_H = 0.0f, my_loss = 0.0f;
  double my_l64 = 0.0;
  int my_kappa = 0;
  bool my_def = false;   // this lane's row was deferred to fwl_overflow_rows
  bool my_unl = false;   // candidate-list mode: this lane's row left unlisted (mark_unlisted)
  double lsum = 0.0;
  auto row_at = [&](int k) { return static_cast<const char*>(z) + (w + (int64_t)k * stride) * o.ld * kElemBytes<T>; };
  // the next row's first round is loaded before this row is resolved (see fwl_block_rows)
  Round<T, V4> first;
  auto first_round = [&](const void* p) {
    const int ws = win_shift<T, MODE, V4>(p);
    stream_first<1, T, V4>(static_cast<const char*>(p) - kElemBytes<T> * ws, C + ws, lane, 0, first);
  };
  if (nrows > 0) first_round(row_at(0));
  for (int k = 0; k < nrows; ++k) {
    const int ku = uniform(k);   // (the compiler keeps the counter in a vector register)
    const int64_t r = w + (int64_t)ku * stride;
    const void* row = row_at(ku);
    const int64_t y64 = ((int64_t)__builtin_amdgcn_readlane((int)(my_y >> 32), k) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane((int)my_y, k);
    const bool yok = y64 >= 0 && y64 < C;
    const int yr = yok ? (int)y64 : -1;

    StreamState st = stream_state(o.force_generic != 0);
    st.sh = win_shift<T, MODE, V4>(row);
    st.ylab = yr >= 0 ? yr + st.sh : -1;   // the label's logit, taken from the stream (window index)
    void* out_row = nullptr;
    if constexpr (MODE == kGrad) out_row = static_cast<char*>(o.grad) + r * (int64_t)C * kElemBytes<T>;
    else if constexpr (MODE == kMask) out_row = o.mask + r * (int64_t)C;
    stream_span<1, T, MODE, V4>(static_cast<const char*>(row) - kElemBytes<T> * st.sh, out_row, C + st.sh, lane, 0,
                                bv, bi, s_w[wid].trash + lane, vcap, icap, st, first);
    if (k + 1 < nrows) first_round(row_at(ku + 1));
    double tau;
    int kappa;
    uint64_t support = 0;
    if (!st.ovf) {
      // keep the entries above the final bound (every support entry is among them)
      const float tb = bound_below_max(st.m);
      pad_list(bv, st.n, lane);
      st.n = list4_compact(bv, bi, st.n, tb, st.noidx, lane);
      pad_list(bv, st.n, lane);
      // every list entry is > st.t (<= tau): the fixed-point steps of a long list start there
      resolve_list<true>(bv, st.n, fmaxf(tb, st.t), st.m, lane, tau, kappa, support);
    } else {
      double ls;
      int lc;
      float lB;
      stream_lower_set(st, bv, lane, ls, lc, lB);
      const float t1 = fmaxf(fmaxf(st.t, bound_below_max(st.m)), safe_lower32(ls, lc, lB));
      if (o.ovf_lo != nullptr) {
        // fwl_overflow_rows solves the row and writes its outputs
        if (lane == 0) {
          o.ovf_lo[r] = t1;
          o.ovf_mx[r] = st.m;
        }
        if (lane == k) my_def = true;
        __builtin_amdgcn_wave_barrier();
        continue;
      }
      select_bisect<1, T, V4, false>(row, C, t1, st.m, sm, lane, 0, tau, kappa);
    }
    if (lane == 0 && !st.ovf && o.ovf_lo != nullptr) o.ovf_lo[r] = NAN;
    const float Hf = rd32(tau);
    const float inv = (float)(o.scale / (double)kappa);
    // this wavefront's zero placeholders have landed before any entry is rewritten (candidate
    // lists have none: the next row's first loads stay in flight)
    if constexpr (MODE != kCand) wait_vmem();
    if (st.noidx && !st.ovf) {
      // the list kept values only: the support from one more pass over the row (candidate lists
      // cut at ccap leave a longer support to fwl_scatter_support, which reads the row itself)
      if (MODE != kCand || (kappa <= o.ccap && !o.mark_unlisted))
        write_support<1, T, MODE, V4, true>(row, r, C, yr, Hf, inv, o, nullptr, lane, 0);
    } else if (!st.ovf) {
      if constexpr (MODE == kGrad || MODE == kMask) {
        for (int p = lane; p < st.n; p += kWave) {
          const int id = bi[p];
          if (id == yr || !(bv[p] > Hf)) continue;
          if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + id, inv);
          else o.mask[r * (int64_t)C + id] = 1;
        }
      } else {
        int out = 0;
        for (int p0 = 0; p0 < st.n; p0 += kWave) {
          const int p = p0 + lane;
          const float v = p < st.n ? bv[p] : -INFINITY;
          const bool sel = v > Hf;
          const uint64_t b = ballot(sel);
          if (sel && out + rank_in(b) < o.ccap) {
            if (o.cval != nullptr) o.cval[r * (int64_t)o.cstride + out + rank_in(b)] = v;
            o.cidx[r * (int64_t)o.cstride + out + rank_in(b)] = bi[p];
          }
          out += __popcll(b);
        }
      }
    } else {
      write_support<1, T, MODE, V4, false>(row, r, C, yr, Hf, inv, o, nullptr, lane, 0);
    }
    const float zy = yok ? st.zy : NAN;
    if (lane == 0 && yok) {
      if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + yr, (zy > Hf ? inv : 0.0f) - o.scale_f);
      else if constexpr (MODE == kMask) o.mask[r * (int64_t)C + yr] = (uint8_t)(zy > Hf);
    }
    const double l64 = (1.0 - (double)zy) + tau;
    const float loss = (float)l64;
    lsum += (double)loss;
    if (lane == k) {
      my_H = Hf;
      my_loss = loss;
      my_l64 = l64;
      my_kappa = kappa;
      my_unl = MODE == kCand && st.noidx && !st.ovf && o.mark_unlisted != 0;
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (lane < nrows && !my_def) {
    const int64_t r = w + (int64_t)lane * stride;
    if (o.H) o.H[r] = my_H;
    if (o.loss) o.loss[r] = my_loss;
    if (o.loss64) o.loss64[r] = my_l64;
    if (o.kappa) o.kappa[r] = my_kappa;
    if constexpr (MODE == kCand) o.ccnt[r] = my_unl ? -my_kappa : my_kappa;
  }
  // each wavefront's loss sum in the first bytes of its own (now unused) list
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) *reinterpret_cast<double*>(s_w[wid].val) = lsum;
  __syncthreads();
  auto wsum = [&](int q) { return *reinterpret_cast<const double*>(s_w[q].val); };
  const double bsum = (wsum(0) + wsum(1)) + (wsum(2) + wsum(3));
  mean_epilogue(bsum, o);
}

// ------------------------------------------------------------------------------------------------
// fwl_overflow_rows: the rows whose candidate lists overflowed in fwl_block_rows or
// fwl_wave_stream_rows (ovf_lo[r] not NaN), one block per row, each solved in memory by
// select_in_memory from the lower bound and maximum the stream left.  The stream wrote the row's
// zero placeholders; this kernel writes its support, its label element, H, loss, kappa and its
// share of the mean (the block partials after those of the streaming kernel).  Launched after
// every streaming launch (it returns at once for rows without overflow).
template <typename T, int MODE, bool V4>
__global__ __launch_bounds__(kBlock) void fwl_overflow_rows(const void* __restrict__ z,
                                                            const int64_t* __restrict__ tgt, int64_t N, int C,
                                                            Outs o) {
  __shared__ BlockShared sh;
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const SelMem sm = {sh.hcnt, sh.hsum, sh.blist, kHistBlock, o.cap * 2 * kWavesPerBlock, sh.red_s, sh.red_c, &sh.ncol};
  double bsum = 0.0;
  // one deferred row, solved by the whole block
  auto solve = [&](int64_t r) {
    const float lo = o.ovf_lo[r];
    const float M = o.ovf_mx[r];
    const void* row = static_cast<const char*>(z) + r * o.ld * kElemBytes<T>;
    const int64_t y64 = tgt[r];
    const bool yok = y64 >= 0 && y64 < C;
    const int yr = yok ? (int)y64 : -1;
    double tau;
    int kappa;
    select_in_memory<kWavesPerBlock, T, V4>(row, C, lo, M, sm, lane, wid, tau, kappa);
    __syncthreads();
    const float Hf = rd32(tau);
    const float inv = (float)(o.scale / (double)kappa);
    // candidate lists cut at ccap (the two-pass op's read pass) leave rows with a longer support
    // to the write pass, which writes them from the logits
    if (MODE != kCand || kappa <= o.ccap)
      write_support<kWavesPerBlock, T, MODE, V4, true>(row, r, C, yr, Hf, inv, o, sh.wsel, lane, wid);
    if (threadIdx.x == 0) {
      const float zy = yok ? load_elem<T>(row, yr) : NAN;
      if (yok) {
        if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + yr, (zy > Hf ? inv : 0.0f) - o.scale_f);
        else if constexpr (MODE == kMask) o.mask[r * (int64_t)C + yr] = (uint8_t)(zy > Hf);
      }
      const double l64 = (1.0 - (double)zy) + tau;
      const float loss = (float)l64;
      if (o.H) o.H[r] = Hf;
      if (o.loss) o.loss[r] = loss;
      if (o.loss64) o.loss64[r] = l64;
      if (o.kappa) o.kappa[r] = kappa;
      if constexpr (MODE == kCand) o.ccnt[r] = kappa;
      bsum += (double)loss;
    }
    __syncthreads();
  };
  // this block's rows are blockIdx.x + j * gridDim.x; their records are read kBlock at a time,
  // one per thread, and only the deferred rows (lower bound not NaN) are solved
  const int64_t nrows = blockIdx.x < N ? (N - 1 - blockIdx.x) / gridDim.x + 1 : 0;
  for (int64_t j0 = 0; j0 < nrows; j0 += kBlock) {
    const int64_t jt = j0 + threadIdx.x;
    const float lt = jt < nrows ? o.ovf_lo[blockIdx.x + jt * gridDim.x] : NAN;
    const uint64_t dm = ballot(lt == lt);
    if (lane == 0) sh.defm[wid] = dm;
    __syncthreads();
    uint64_t pend[kWavesPerBlock];
#pragma unroll
    for (int q = 0; q < kWavesPerBlock; ++q) pend[q] = sh.defm[q];
    __syncthreads();
    for (int q = 0; q < kWavesPerBlock; ++q) {
      while (pend[q] != 0) {
        const int64_t j = j0 + kWave * q + __builtin_ctzll(pend[q]);
        pend[q] &= pend[q] - 1;
        solve(uniform64(blockIdx.x + j * gridDim.x));   // (pend comes from LDS)
      }
    }
  }
  mean_epilogue(bsum, o);
}

// ------------------------------------------------------------------------------------------------
// Split rows: few rows, each very long.  fwl_split_chunks runs one block per (row, chunk): it
// streams the chunk (zero placeholders, candidate lists), resolves the chunk's own threshold
// tau_c and keeps the chunk's own support, {z > tau_c} -- tau_c = H(top kappa_c of the chunk) <=
// tau, so the row's support lies in the union of the chunk supports.  fwl_split_finish runs one
// block per row on that union: every entry above max_c tau_c, resolved like a candidate list.
// A chunk whose support exceeds kSplitCap entries (or whose lists overflow) marks its row for the
// generic solve, which the finishing kernel runs on the row in memory.

constexpr int kSplitCap = 64;           // support entries kept per chunk
// measured on MI355X (fp32, 1..256 rows of 16384..128256): splitting wins up to 128 rows of at
// least ~96 KiB (1.3-2.9x at 1..64 rows of 128256); one block per row wins beyond
constexpr int kSplitMaxRows = 128;      // rows up to which long rows are split
constexpr int64_t kSplitMinBytes = 96 * 1024;   // shortest row (in bytes) that is split
constexpr int kSplitTargetItems = 1024; // (row, chunk) items to aim for
constexpr int kSplitMinChunk = 4096;    // elements: one streaming round of a block (fp32)
constexpr int kSplitMaxChunks = 256;
constexpr int kSplitListCap = 2048;     // entries of a row's list in the finishing kernel

struct SplitScratch {
  int* count;     // [N * nch]: support size of the chunk, -1 = the row needs the overflow solve
  double* tau;    // [N * nch]: tau_c, or a lower bound on tau where count = -1
  float* mx;      // [N * nch]: the chunk's maximum
  float* val;     // [N * nch * kSplitCap]
  int* idx;       // [N * nch * kSplitCap] (index within the row)
};

template <typename T, int MODE, bool V4>
__global__ __launch_bounds__(kBlock) void fwl_split_chunks(const void* __restrict__ z, int64_t N, int C, int CH,
                                                           int nch, Outs o, SplitScratch sc) {
  __shared__ BlockShared sh;
  __shared__ int s_base[kWavesPerBlock];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t items = N * (int64_t)nch;
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int64_t r = it / nch;
    const int c = (int)(it - r * nch);
    const int c0 = c * CH;
    const int len = C - c0 < CH ? C - c0 : CH;
    const void* span = static_cast<const char*>(z) + (r * o.ld + c0) * kElemBytes<T>;
    void* out_span = nullptr;
    if constexpr (MODE == kGrad) out_span = static_cast<char*>(o.grad) + (r * (int64_t)C + c0) * kElemBytes<T>;
    else if constexpr (MODE == kMask) out_span = o.mask + r * (int64_t)C + c0;
    float* bv = sh.bval[wid];
    int* bi = sh.bidx[wid];
    StreamState st = stream_state(o.force_generic != 0);
    Round<T, V4> first;
    stream_first<kWavesPerBlock, T, V4>(span, len, lane, wid, first);
    stream_span<kWavesPerBlock, T, MODE, V4>(span, out_span, len, lane, wid, bv, bi, sh.trash[wid] + lane, o.cap,
                                             o.cap, st, first);
    if (lane == 0) {
      sh.wmax[wid] = st.m;
      sh.wn[wid] = st.n;
      sh.ovf[wid] = st.ovf;
    }
    __syncthreads();
    const bool overflow = sh.ovf[0] | sh.ovf[1] | sh.ovf[2] | sh.ovf[3];
    const float Mc = fmaxf(fmaxf(sh.wmax[0], sh.wmax[1]), fmaxf(sh.wmax[2], sh.wmax[3]));
    // the chunk's support, {list entries > rd32(tau_c)}, or -1: the row needs the overflow solve
    // (lists overflowed; a support too large to keep; a +inf maximum, whose row has no finite
    // tau).  tau_c (or, after an overflow, H of the entries the stream summed, a lower bound) is
    // kept either way: the largest over the chunks is where the row's solve starts.
    int status = -1;
    double lower = -INFINITY;
    if (!overflow) {
      block_merge_resolve(sh, st.n, wid, lane);
      __syncthreads();
      if (sh.kappa == 0) {
        status = Mc == -INFINITY ? 0 : -1;   // 0: no finite entry in the chunk
      } else if (isfinite(sh.tau)) {
        lower = sh.tau;
        const float Hc = rd32(sh.tau);
        int cnt = 0;
        for (int p0 = 0; p0 < st.n; p0 += kWave) cnt += __popcll(ballot(p0 + lane < st.n && bv[p0 + lane] > Hc));
        if (lane == 0) s_base[wid] = cnt;
        __syncthreads();
        const int total = (s_base[0] + s_base[1]) + (s_base[2] + s_base[3]);
        if (total <= kSplitCap) {
          status = total;
          int off = 0;
          for (int w = 0; w < wid; ++w) off += s_base[w];
          const int64_t slot = it * kSplitCap;
          for (int p0 = 0; p0 < st.n; p0 += kWave) {
            const int p = p0 + lane;
            const bool sel = p < st.n && bv[p] > Hc;
            const uint64_t b = ballot(sel);
            if (sel) {
              sc.val[slot + off + rank_in(b)] = bv[p];
              sc.idx[slot + off + rank_in(b)] = c0 + bi[p];
            }
            off += __popcll(b);
          }
        }
      }
    } else {
      double ls;
      int lc;
      float lB;
      stream_lower_set(st, bv, lane, ls, lc, lB);
      if (lane == 0) {
        sh.wlo[wid] = st.t;
        sh.wB[wid] = lB;
        sh.red_s[wid] = ls;
        sh.red_c[wid] = lc;
      }
      __syncthreads();
      const double S = (sh.red_s[0] + sh.red_s[1]) + (sh.red_s[2] + sh.red_s[3]);
      const int Cn = (sh.red_c[0] + sh.red_c[1]) + (sh.red_c[2] + sh.red_c[3]);
      const float B = fmaxf(fmaxf(sh.wB[0], sh.wB[1]), fmaxf(sh.wB[2], sh.wB[3]));
      lower = fmaxf(fmaxf(fmaxf(sh.wlo[0], sh.wlo[1]), fmaxf(sh.wlo[2], sh.wlo[3])), safe_lower32(S, Cn, B));
    }
    if (threadIdx.x == 0) {
      sc.count[it] = status;
      sc.tau[it] = status > 0 || status < 0 ? lower : -INFINITY;
      sc.mx[it] = Mc;
    }
    __syncthreads();
  }
}

// One block per row.  Thread t reads chunk t's bound and support; the entries above the largest
// chunk bound form the row's list in LDS (chunk order), which wavefront 0 resolves.
template <typename T, int MODE, bool V4>
__global__ __launch_bounds__(kBlock) void fwl_split_finish(const void* __restrict__ z, const int64_t* __restrict__ tgt,
                                                           int64_t N, int C, int nch, Outs o, SplitScratch sc) {
  static_assert(kSplitMaxChunks <= kBlock, "one thread per chunk");
  static_assert(kSplitListCap <= kWavesPerBlock * kCapMax, "the row's list lives in the block's candidate lists");
  constexpr int B = 8;   // support entries loaded per batch
  __shared__ BlockShared sh;
  __shared__ double s_lo[kWavesPerBlock];
  __shared__ float s_mx[kWavesPerBlock];
  __shared__ int s_w[kWavesPerBlock];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int t = (int)threadIdx.x;
  float* cl = &sh.bval[0][0];
  int* cx = &sh.bidx[0][0];
  double lsum = 0.0;
  const SelMem sm = {sh.hcnt, sh.hsum, sh.blist, kHistBlock, o.cap * 2 * kWavesPerBlock, sh.red_s, sh.red_c, &sh.ncol};
  for (int64_t r = blockIdx.x; r < N; r += gridDim.x) {
    const void* row = static_cast<const char*>(z) + r * o.ld * kElemBytes<T>;
    const int64_t y64 = tgt[r];
    // the chunks' lower bounds, and whether any chunk gave up
    const int64_t item = r * nch + t;
    const int cnt = t < nch ? sc.count[item] : 0;
    const double tc = t < nch ? sc.tau[item] : -INFINITY;
    const float mc = t < nch ? sc.mx[item] : -INFINITY;
    const bool yok = y64 >= 0 && y64 < C;
    const int yr = yok ? (int)y64 : -1;
    const float zy = t == 0 && yok ? load_elem<T>(row, yr) : NAN;   // used by thread 0
    const double wlo = wave_max_f64(tc);
    const float wmx = wave_max_f32(mc);
    const int wbad = ballot(cnt < 0) != 0;
    if (lane == 0) {
      s_lo[wid] = wlo;
      s_mx[wid] = wmx;
      s_w[wid] = wbad;
    }
    __syncthreads();
    const double lo = fmax(fmax(s_lo[0], s_lo[1]), fmax(s_lo[2], s_lo[3]));
    const float Mrow = fmaxf(fmaxf(s_mx[0], s_mx[1]), fmaxf(s_mx[2], s_mx[3]));
    bool generic = ((s_w[0] | s_w[1]) | (s_w[2] | s_w[3])) != 0 || o.force_generic;
    __syncthreads();
    // chunk t's entries above lo: count them, then write them at their place in the row's list
    // (the first B entries stay in registers; longer chunk supports are read again)
    const float lof = rd32(lo);
    const int64_t slot = item * kSplitCap;
    int mine = 0;
    float v0[B];
    int id0[B];
#pragma unroll
    for (int k = 0; k < B; ++k) {
      const bool in = !generic && k < cnt;
      v0[k] = in ? sc.val[slot + k] : -INFINITY;
      id0[k] = in ? sc.idx[slot + k] : 0;
      mine += v0[k] > lof;
    }
    if (!generic) {
      for (int e0 = B; e0 < cnt; e0 += B) {
        float v[B];
#pragma unroll
        for (int k = 0; k < B; ++k) v[k] = e0 + k < cnt ? sc.val[slot + e0 + k] : -INFINITY;
#pragma unroll
        for (int k = 0; k < B; ++k) mine += v[k] > lof;
      }
    }
    int wtot;
    int off = wave_excl_scan_i32(mine, wtot);
    if (lane == 0) s_w[wid] = wtot;
    __syncthreads();
    for (int w = 0; w < wid; ++w) off += s_w[w];
    const int n = (s_w[0] + s_w[1]) + (s_w[2] + s_w[3]);
    generic = generic || n > kSplitListCap;
    if (!generic && mine > 0) {
#pragma unroll
      for (int k = 0; k < B; ++k) {
        if (v0[k] > lof) {
          cl[off] = v0[k];
          cx[off] = id0[k];
          ++off;
        }
      }
      for (int e0 = B; e0 < cnt; e0 += B) {
        float v[B];
        int id[B];
#pragma unroll
        for (int k = 0; k < B; ++k) {
          const bool in = e0 + k < cnt;
          v[k] = in ? sc.val[slot + e0 + k] : -INFINITY;
          id[k] = in ? sc.idx[slot + e0 + k] : 0;
        }
#pragma unroll
        for (int k = 0; k < B; ++k) {
          if (v[k] > lof) {
            cl[off] = v[k];
            cx[off] = id[k];
            ++off;
          }
        }
      }
    }
    __syncthreads();
    double tau;
    int kappa;
    if (!generic) {
      if (wid == 0) {
        float lm = -INFINITY;
        for (int p = lane; p < n; p += kWave) lm = fmaxf(lm, cl[p]);
        double tt;
        int kk;
        uint64_t sup;
        resolve_list(cl, n, lof, wave_max_f32(lm), lane, tt, kk, sup);
        if (lane == 0) {
          sh.tau = tt;
          sh.kappa = kk;
        }
      }
      __syncthreads();
      tau = sh.tau;
      kappa = sh.kappa;
      const float Hf = rd32(tau);
      const float inv = (float)(o.scale / (double)kappa);
      // the support (every other output element holds the zero placeholder already)
      if constexpr (MODE == kGrad || MODE == kMask) {
        for (int p = t; p < n; p += kBlock) {
          const int id = cx[p];
          if (id == yr || !(cl[p] > Hf)) continue;
          if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + id, inv);
          else o.mask[r * (int64_t)C + id] = 1;
        }
      } else {
        int base = 0;
        for (int p0 = 0; p0 < n; p0 += kBlock) {
          const int p = p0 + t;
          const float v = p < n ? cl[p] : -INFINITY;
          const bool sel = v > Hf;
          const uint64_t b = ballot(sel);
          if (lane == 0) sh.wsel[wid] = __popcll(b);
          __syncthreads();
          int q = base;
          for (int w = 0; w < wid; ++w) q += sh.wsel[w];
          if (sel && q + rank_in(b) < o.ccap) {
            o.cval[r * (int64_t)o.cstride + q + rank_in(b)] = v;
            o.cidx[r * (int64_t)o.cstride + q + rank_in(b)] = cx[p];
          }
          base += (sh.wsel[0] + sh.wsel[1]) + (sh.wsel[2] + sh.wsel[3]);
          __syncthreads();
        }
      }
    } else {
      // every chunk bound is a lower bound on tau (tau_c of a subset, or H of summed entries)
      const float t1 = fmaxf(rd32(lo), bound_below_max(Mrow));
      select_in_memory<kWavesPerBlock, T, V4>(row, C, t1, Mrow, sm, lane, wid, tau, kappa);
      __syncthreads();
      write_support<kWavesPerBlock, T, MODE, V4, true>(row, r, C, yr, rd32(tau), (float)(o.scale / (double)kappa), o,
                                                       sh.wsel, lane, wid);
    }
    if (t == 0) {
      const float Hf = rd32(tau);
      const float inv = (float)(o.scale / (double)kappa);
      if (yok) {
        if constexpr (MODE == kGrad) store_elem<T>(o.grad, r * (int64_t)C + yr, (zy > Hf ? inv : 0.0f) - o.scale_f);
        else if constexpr (MODE == kMask) o.mask[r * (int64_t)C + yr] = (uint8_t)(zy > Hf);
      }
      const double l64 = (1.0 - (double)zy) + tau;
      const float loss = (float)l64;
      if (o.H) o.H[r] = Hf;
      if (o.loss) o.loss[r] = loss;
      if (o.loss64) o.loss64[r] = l64;
      if (o.kappa) o.kappa[r] = kappa;
      if constexpr (MODE == kCand) o.ccnt[r] = kappa;
      lsum += (double)loss;
    }
    __syncthreads();
  }
  mean_epilogue(lsum, o);
}

// ------------------------------------------------------------------------------------------------
// two-op backward kernels of the drop-in interface

// grad = (mask ? inv : 0) - [j == y] * scale, one wavefront per row (rows w + k*stride, k < 64).
// The gradient stores carry no non-temporal hint (measured at cfg2, two-op sequence 132 -> 118 us;
// the mask loads keep it).
// The wavefront's rows form one sequence of rounds (kMaskSlots mask units per lane, a unit being 4
// mask bytes and 16 gradient bytes, or 1 and 4 for rows that are not 16-byte aligned); the mask
// loads of the next round are issued before the gradient stores of the current one.
constexpr int kMaskSlots = 4;

template <bool V4>
__device__ __forceinline__ void mask_round_load(rsrc_t m, int round, int lane, uint32_t* mk) {
#pragma unroll
  for (int u = 0; u < kMaskSlots; ++u) {
    const uint32_t q = (uint32_t)(round * kWave * kMaskSlots + lane + kWave * u);
    if constexpr (V4) mk[u] = __builtin_amdgcn_raw_buffer_load_b32(m, 4u * q, 0, kNonTemporal);
    else mk[u] = __builtin_amdgcn_raw_buffer_load_b8(m, q, 0, kNonTemporal);
  }
}

template <bool V4>
__device__ __forceinline__ void mask_round_store(rsrc_t g, int round, int lane, const uint32_t* mk, int yr,
                                                 uint32_t b_inv, uint32_t b_lab_in, uint32_t b_lab_out) {
#pragma unroll
  for (int u = 0; u < kMaskSlots; ++u) {
    const int q = round * kWave * kMaskSlots + lane + kWave * u;
    if constexpr (V4) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool sel = ((mk[u] >> (8 * e)) & 0xFFu) != 0u;
        w[e] = 4 * q + e == yr ? (sel ? b_lab_in : b_lab_out) : (sel ? b_inv : 0u);
      }
      __builtin_amdgcn_raw_buffer_store_b128(v4u{w[0], w[1], w[2], w[3]}, g, 16u * (uint32_t)q, 0, 0);
    } else {
      const bool sel = (mk[u] & 0xFFu) != 0u;
      const uint32_t w = q == yr ? (sel ? b_lab_in : b_lab_out) : (sel ? b_inv : 0u);
      __builtin_amdgcn_raw_buffer_store_b32(w, g, 4u * (uint32_t)q, 0, 0);
    }
  }
}

template <bool V4>
__global__ __launch_bounds__(kBlock) void fwl_mask_to_grad(const int64_t* __restrict__ tgt,
                                                           const uint8_t* __restrict__ mask,
                                                           const int32_t* __restrict__ kap,
                                                           int64_t N, int C, double scale,
                                                           float scale_f, float* __restrict__ grad) {
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  const int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wid;
  const int nrows = w < N ? (int)((N - 1 - w) / stride + 1) : 0;   // <= kRowsPerWave (host grid)
  const int units = V4 ? C / 4 : C;
  const int rounds = (units + kWave * kMaskSlots - 1) / (kWave * kMaskSlots);
  const int64_t my_y = lane < nrows ? tgt[w + (int64_t)lane * stride] : 0;
  const int my_kap = lane < nrows ? kap[w + (int64_t)lane * stride] : 0;
  auto mask_rsrc = [&](int k) {
    return k < nrows ? make_rsrc(mask + (w + (int64_t)k * stride) * C, (uint32_t)C) : make_rsrc(mask, 0u);
  };
  if (nrows == 0) return;
  const int items = nrows * rounds;   // (row, round) pairs, row-major
  uint32_t mk[kMaskSlots];
  mask_round_load<V4>(mask_rsrc(0), 0, lane, mk);
  __builtin_amdgcn_sched_barrier(0);   // mirror of the loop's stores (see mirror_row_stores)
  {
    uint32_t zero[kMaskSlots] = {};
    mask_round_store<V4>(make_rsrc(nullptr, 0u), 0, lane, zero, -1, 0u, 0u, 0u);
  }
  __builtin_amdgcn_sched_barrier(0);
  int it = 0;
  do {
    const int k = it / rounds, rd = it - k * rounds;
    const int kn = (it + 1) / rounds, rdn = it + 1 - kn * rounds;
    uint32_t cur[kMaskSlots];
#pragma unroll
    for (int u = 0; u < kMaskSlots; ++u) cur[u] = mk[u];
    mask_round_load<V4>(it + 1 < items ? mask_rsrc(kn) : make_rsrc(mask, 0u), rdn, lane, mk);
    const int64_t y = ((int64_t)__builtin_amdgcn_readlane((int)(my_y >> 32), k) << 32) |
                      (uint32_t)__builtin_amdgcn_readlane((int)my_y, k);
    const int yr = (y >= 0 && y < C) ? (int)y : -1;
    const float inv = (float)(scale / (double)__builtin_amdgcn_readlane(my_kap, k));
    const rsrc_t g = make_rsrc(grad + (w + (int64_t)k * stride) * C, 4u * (uint32_t)C);
    mask_round_store<V4>(g, rd, lane, cur, yr, __float_as_uint(inv), __float_as_uint(inv - scale_f),
                         __float_as_uint(0.0f - scale_f));
  } while (++it < items);
}

template <bool V4>
__global__ __launch_bounds__(kBlock) void fwl_cand_to_grad(
    const float* __restrict__ z, const int64_t* __restrict__ tgt, const float* __restrict__ Hin,
    const int32_t* __restrict__ kap, const float* __restrict__ cval, const int32_t* __restrict__ cidx,
    const int32_t* __restrict__ ccnt, int64_t N, int C, double scale, float scale_f,
    float* __restrict__ grad) {
  for (int64_t r = blockIdx.x; r < N; r += gridDim.x) {
    float* gr = grad + r * (int64_t)C;
    if constexpr (V4) {
      const int nvec = C >> 2;
      for (int q = threadIdx.x; q < nvec; q += kBlock)
        __builtin_nontemporal_store(v4f{0.0f, 0.0f, 0.0f, 0.0f}, reinterpret_cast<v4f*>(gr) + q);
    } else {
      for (int j = threadIdx.x; j < C; j += kBlock) __builtin_nontemporal_store(0.0f, gr + j);
    }
    // the zeros must land before the scattered values below (same addresses, other threads of
    // this block, hence the same L2)
    wait_vmem();
    __syncthreads();
    const int64_t y64 = tgt[r];
    const int yr = (y64 >= 0 && y64 < C) ? (int)y64 : -1;
    const float h = Hin[r];
    const float inv = (float)(scale / (double)kap[r]);
    int cnt = ccnt[r];
    cnt = cnt < 0 ? 0 : (cnt > C ? C : cnt);
    for (int p = threadIdx.x; p < cnt; p += kBlock) {
      const float v = cval[r * (int64_t)C + p];
      const int id = cidx[r * (int64_t)C + p];
      if (id >= 0 && id < C && id != yr && v > h) gr[id] = inv;
    }
    if (threadIdx.x == 0 && yr >= 0) gr[yr] = (z[r * (int64_t)C + yr] > h ? inv : 0.0f) - scale_f;
    __syncthreads();
  }
}

// Write pass of the fused op for long rows.  A read pass over the logits (the candidate-list
// kernel, its lists cut at kTwoPassCap indices in the workspace) leaves every row's H, kappa and,
// where its list kept the indices, its support.  The gradient is then written by two kernels:
// fwl_fill_zero streams zeros over the whole [N, C] gradient in 4 KB blocks, a plain fill that
// needs nothing from the read pass; then fwl_scatter_support writes each row's listed support
// entries and its label element (one wavefront per row).  Rows whose support is not listed are
// rewritten from the logits (z > H).  Measured on MI355X: a 1 GiB fill writes at 6.8 TB/s in
// 4 KB blocks but at 6.1 TB/s in 16 KB blocks, and a block that must first load its row's data
// before storing is bound by that latency.
constexpr int kTwoPassCap = kCapMax;     // support indices kept per row between the passes

// the read pass's per-row count: kappa where the support is listed, -kappa (or a kappa above
// kTwoPassCap) where it is not
__device__ __forceinline__ bool two_pass_listed(int k) { return k > 0 && k <= kTwoPassCap; }
__device__ __forceinline__ int two_pass_kappa(int k) { return k < 0 ? -k : k; }
constexpr int kTwoPassWaveRowsPerCU = 8;    // rows per CU from which the read pass takes a wavefront per row
constexpr int64_t kTwoPassMinCWin16 = 12000;   // 16-bit rows without 128-bit units: two passes from this length
constexpr int kFillBytes = 4096;         // bytes per block of the fill

// kap (optional): per row the read pass's count; rows whose support is not listed are left alone
// (the scatter writes them whole).  Needs rows of a whole number of dwords and of >= kFillBytes bytes, so that a
// block's bytes lie in at most two rows and no dword straddles two rows.
__global__ __launch_bounds__(kBlock) void fwl_fill_zero(void* __restrict__ dst, int64_t bytes, int64_t row_bytes,
                                                         const int32_t* __restrict__ kap) {
  const int64_t b0 = (int64_t)blockIdx.x * kFillBytes;
  const int64_t left = bytes - b0;
  const rsrc_t r = make_rsrc(static_cast<char*>(dst) + b0, (uint32_t)(left < kFillBytes ? left : kFillBytes));
  const uint32_t off = 16u * threadIdx.x;
  if (kap != nullptr) {
    // the block's first row and where the next one starts (block-uniform)
    const int64_t ra = b0 / row_bytes;
    const int64_t next = (ra + 1) * row_bytes - b0;   // bytes into the block
    const bool fa = two_pass_listed(kap[ra]);
    const bool fb = next < kFillBytes && next < left ? two_pass_listed(kap[ra + 1]) : fa;
    if (!fa && !fb) return;
    if (!(fa && fb)) {
      // dwords of the rows to fill only
#pragma unroll
      for (uint32_t d = 0; d < 4; ++d) {
        const uint32_t o4 = off + 4u * d;
        if ((int64_t)o4 < next ? fa : fb) __builtin_amdgcn_raw_buffer_store_b32(0u, r, o4, 0, 0);
      }
      return;
    }
  }
  // 16 bytes per thread; the range check drops what lies past the end (per dword; the caller
  // pads nothing, so a gradient whose size is not a multiple of 4 bytes gets its last 2 bytes
  // from fwl_scatter_support)
  __builtin_amdgcn_raw_buffer_store_b128(v4u{0u, 0u, 0u, 0u}, r, off, 0, 0);
}

// how fwl_scatter_support treats rows whose support is not listed
constexpr int kLongScan = 0;    // the fill wrote their zeros: their support entries from the logits
constexpr int kLongDense = 1;   // the fill left them alone: rewritten whole from the logits
constexpr int kLongDone = 2;    // fwl_write_flat wrote them whole

template <typename T, bool V4>
__global__ __launch_bounds__(kBlock) void fwl_scatter_support(
    const void* __restrict__ z, int64_t ld, const int64_t* __restrict__ tgt, const float* __restrict__ Hin,
    const int32_t* __restrict__ kap_in, const int32_t* __restrict__ cidx, int64_t N, int C, double scale,
    float scale_f, void* __restrict__ grad, bool odd_tail, int dense) {
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid; r < N; r += stride) {
    const bool listed = two_pass_listed(kap_in[r]);
    const int kap = two_pass_kappa(kap_in[r]);
    if (!listed && dense == kLongDone) continue;   // written whole by fwl_write_flat
    const float Hf = Hin[r];
    const int64_t y64 = tgt[r];
    const int yr = (y64 >= 0 && y64 < C) ? (int)y64 : -1;
    const float inv = (float)(scale / (double)kap);
    const void* row = static_cast<const char*>(z) + r * ld * kElemBytes<T>;
    const int64_t g0 = r * (int64_t)C;
    if (listed) {
      for (int p = lane; p < kap; p += kWave) {
        const int id = cidx[r * (int64_t)kTwoPassCap + p];
        if (id != yr) store_elem<T>(grad, g0 + id, inv);
      }
    } else if (dense) {
      // a support longer than the list, on a row the fill left alone: the whole row from the
      // logits (z > H ? inv : 0) in 128-bit units, each line written once, two rounds in flight
      constexpr int PER = Round<T, V4>::kPer;
      constexpr int U = kUnit<T, V4>;
      constexpr int per_round = kWave * Round<T, V4>::kSlots;
      const int rounds = (C + per_round - 1) / per_round;
      const rsrc_t in = make_rsrc_u(row, (uint32_t)(kElemBytes<T> * C));
      const rsrc_t none = make_rsrc_u(row, 0u);
      const rsrc_t out = make_rsrc(static_cast<char*>(grad) + g0 * kElemBytes<T>, (uint32_t)(kElemBytes<T> * C));
      const uint32_t b_inv = encode<T>(inv);
      auto emit = [&](const Round<T, V4>& a, int k) {
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          uint32_t bits[U];
#pragma unroll
          for (int e = 0; e < U; ++e) bits[e] = a.x[U * u + e] > Hf ? b_inv : 0u;
          store_unit_bits<T, V4>(out, (uint32_t)lane_unit<1, PER>(k, u, 0, lane), bits);
        }
      };
      Round<T, V4> a, b;
      load_round<1, T, V4>(in, 0, 0, lane, a);
      for (int k = 0; k < rounds; k += 2) {
        load_round<1, T, V4>(k + 1 < rounds ? in : none, k + 1, 0, lane, b);
        emit(a, k);
        if (k + 1 >= rounds) break;
        load_round<1, T, V4>(k + 2 < rounds ? in : none, k + 2, 0, lane, a);
        emit(b, k + 1);
      }
      wait_vmem();   // the label element below is stored over its value here
    } else if constexpr (!V4 && kElemBytes<T> == 2) {
      // a support longer than the list, 16-bit row without 128-bit units: its entries from the
      // logits (the fill wrote the zeros), streamed with 128-bit loads through a window from the
      // 4-byte boundary below the row (see win_shift), two rounds in flight
      const int ws = (int)((reinterpret_cast<uintptr_t>(row) >> 1) & 1);
      row_pass<1, T, true, true>(static_cast<const char*>(row) - kElemBytes<T> * ws, C + ws, lane, 0,
                                 [&](float zj, int jw) {
                                   const int j = jw - ws;
                                   if (j >= 0 && zj > Hf && j != yr) store_elem<T>(grad, g0 + j, inv);
                                 });
    } else {
      // a support longer than the list: its entries from the logits (the fill wrote the zeros),
      // the row streamed in 128-bit units with two rounds in flight
      row_pass<1, T, V4, true>(row, C, lane, 0, [&](float zj, int j) {
        if (zj > Hf && j != yr) store_elem<T>(grad, g0 + j, inv);
      });
    }
    if (lane == 0) {
      if (yr >= 0) store_elem<T>(grad, g0 + yr, (load_elem<T>(row, yr) > Hf ? inv : 0.0f) - scale_f);
      // a 16-bit gradient of odd size: its last element lies past the fill's last whole dword
      if (odd_tail && r == N - 1 && yr != C - 1) {
        const float zl = load_elem<T>(row, C - 1);
        store_elem<T>(grad, g0 + C - 1, zl > Hf ? inv : 0.0f);
      }
    }
  }
}

// fwl_write_flat: the two-pass op's gradient for rows of a whole number of 128-bit units, one
// block per 4 KB of the [N, C] gradient, one 128-bit unit per thread, stored once:
//   * rows whose support the read pass listed: zeros (fwl_scatter_support then stores the listed
//     support entries and the label element);
//   * other rows: the unit's logits are loaded and inv stored where z > H; the label element
//     gets its scale subtracted in the same store.
// Measured on MI355X over 1 GiB: zero stores reach 6.85 TB/s in 4 KB blocks of 256 threads, 6.80
// with a load from a small cached array before them, against 5.5-5.8 TB/s from resident
// wavefronts looping over items; stores that first load the logits under them move 6.1 TB/s of
// read and write traffic together (8 KB and 16 KB blocks: less).  A row's kappa comes through the
// scalar cache, so a block's only wait on memory before its stores is that of its logits.
constexpr int kWriteBytes = 4096;   // gradient bytes per block

template <typename T>
__global__ __launch_bounds__(kBlock) void fwl_write_flat(
    const void* __restrict__ z, int64_t ld, const int64_t* __restrict__ tgt, const float* __restrict__ Hin,
    const int32_t* __restrict__ kap_in, int64_t N, int C, double scale, float scale_f, void* __restrict__ grad) {
  constexpr int U = kUnit<T, true>;
  const int64_t units = N * (int64_t)(C / U);
  const int64_t u0 = (int64_t)blockIdx.x * (kWriteBytes / 16);   // the block's first unit
  const int64_t ug = u0 + threadIdx.x;
  if (ug >= units) return;
  // the unit's row and its index q within the row (rows are whole units)
  const int upr = C / U;
  const int64_t rb = u0 / upr;   // the block's first row
  const int du = (int)(ug - rb * upr);
  const int64_t r = rb + du / upr;
  const int q = du % upr;
  // kappa of the block's first two rows through the scalar cache (a block spans at most two rows
  // of >= 4 KB), of others per thread
  const int kap0 = kap_in[rb];
  const int kap1 = rb + 1 < N ? kap_in[rb + 1] : 0;
  const int kc = r == rb ? kap0 : (r == rb + 1 ? kap1 : kap_in[r]);
  const rsrc_t out = make_rsrc(static_cast<char*>(grad) + u0 * 16, (uint32_t)kWriteBytes);
  if (two_pass_listed(kc)) {
    store_zero_unit<T, true>(out, threadIdx.x);
    return;
  }
  const int kap = two_pass_kappa(kc);
  float x[U];
  const rsrc_t in = make_rsrc(static_cast<const char*>(z) + r * ld * kElemBytes<T>, (uint32_t)(kElemBytes<T> * C));
  load_unit<T, true>(in, (uint32_t)q, x);
  const float Hf = Hin[r];
  const int64_t y64 = tgt[r];
  const int yr = (y64 >= 0 && y64 < C) ? (int)y64 : -1;
  const float inv = (float)(scale / (double)kap);
  const uint32_t b_inv = encode<T>(inv);
  uint32_t bits[U];
#pragma unroll
  for (int e = 0; e < U; ++e) {
    const bool sup = x[e] > Hf;
    bits[e] = sup ? b_inv : 0u;
    if (U * q + e == yr) bits[e] = encode<T>((sup ? inv : 0.0f) - scale_f);
  }
  store_unit_bits<T, true, 0>(out, threadIdx.x, bits);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void fwl_scale_rows(void* __restrict__ grad,
                                                         const float* __restrict__ go,
                                                         int64_t go_stride, int64_t N, int C) {
  constexpr int U = kUnit<T, VEC>;
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  const int units = (C + U - 1) / U;
  for (int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid; r < N; r += stride) {
    const float s = go[r * go_stride];
    if (s == 1.0f) continue;
    const rsrc_t row = make_rsrc(static_cast<char*>(grad) + r * (int64_t)C * kElemBytes<T>,
                                 (uint32_t)(kElemBytes<T> * C));
    for (int u = lane; u < units; u += kWave) {
      float v[U];
      load_unit<T, VEC>(row, (uint32_t)u, v);
#pragma unroll
      for (int e = 0; e < U; ++e) v[e] *= s;
      store_unit<T, VEC>(row, (uint32_t)u, v);
    }
  }
}

__global__ void fwl_empty_mean(float* mean, double reduce_div) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *mean = (float)(0.0 / reduce_div);
}

// ------------------------------------------------------------------------------------------------
// host side

// Dispatch switches of one call (fwl_options); the process-wide defaults are set by fwl_set_params.
struct Params {
  int path;         // 0 automatic; 1-8 forced (fwl_set_params)
  int cap;          // LDS candidate capacity per wavefront of the streaming kernels
  bool no_window;   // path 8: path 1 without line-aligned windows
};

std::atomic<int> g_path{0};
std::atomic<int> g_cap{kCapMax};

Params default_params() {
  Params p;
  p.path = g_path.load(std::memory_order_relaxed);
  p.cap = g_cap.load(std::memory_order_relaxed);
  p.no_window = p.path == 8;
  return p;
}

// the call's switches: opt (validated) or the process defaults
bool call_params(const fwl_options* opt, Params& p) {
  p = default_params();
  if (opt == nullptr) return true;
  if (opt->path < 0 || opt->path > 8) return false;
  if (opt->cand_cap != 0 && (opt->cand_cap < kWave || opt->cand_cap > kCapMax)) return false;
  p.path = opt->path;
  p.no_window = opt->path == 8;
  p.cap = opt->cand_cap != 0 ? opt->cand_cap : kCapMax;
  return true;
}

int blocks_row(int64_t N) { return (int)(N < kMaxBlocksRow ? (N > 0 ? N : 1) : kMaxBlocksRow); }

// Blocks of `kernel` that fit on the current device at once (cached per device and kernel).
int resident_blocks(const void* kernel) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(dev, kernel);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kBlock, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const int nb = per_cu * cus;
  cache.emplace(key, nb);
  return nb;
}

// Persistent grid: at most one resident set of blocks (and at most `cap`), with the rows spread
// so that every unit of work (wavefront or block) gets the same number of rows, +-1 at the end.
int persistent_grid(int64_t units, int units_per_block, int resident, int cap) {
  int64_t max_blocks = resident > 0 ? (resident < cap ? resident : cap) : cap;
  const int64_t max_units = max_blocks * units_per_block;
  const int64_t per_unit = (units + max_units - 1) / max_units;
  const int64_t used = (units + per_unit - 1) / per_unit;
  const int64_t blocks = (used + units_per_block - 1) / units_per_block;
  return (int)(blocks > 0 ? blocks : 1);
}

int device_cus() {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
  cache.emplace(dev, cus);
  return cus;
}

// Grid of fwl_wave_rows.  Each wavefront keeps one row load and one row of stores in flight, so
// the blocks per CU set the number of concurrent row streams.  Measured on MI355X with 4000-byte
// rows: two blocks per CU (8 wavefronts, ~64 KB in flight per CU) stream best; more concurrent
// streams over a wider address window lose DRAM efficiency.  Shorter rows (in bytes) get
// proportionally more blocks, up to the resident limit; longer rows at least min_per_cu blocks.
// At most kRowsPerWave rows per wavefront: larger N gets more (queued) blocks.
int wave_grid(int64_t N, int64_t row_bytes, int resident, int min_per_cu = 2) {
  const int cus = device_cus();
  const int per_cu_resident = cus > 0 && resident > 0 ? resident / cus : 0;
  int per_cu = (int)((8000 + row_bytes - 1) / (row_bytes > 0 ? row_bytes : 1));
  if (per_cu < min_per_cu) per_cu = min_per_cu;
  if (per_cu_resident > 0 && per_cu > per_cu_resident) per_cu = per_cu_resident;
  const int target = cus > 0 ? per_cu * cus : (resident > 0 ? resident : kMaxBlocksWave);
  const int64_t min_blocks = (N + (int64_t)kWavesPerBlock * kRowsPerWave - 1) / ((int64_t)kWavesPerBlock * kRowsPerWave);
  const int cap = (int)(min_blocks > kMaxBlocksWave ? min_blocks : kMaxBlocksWave);
  const int64_t g = persistent_grid(N, kWavesPerBlock, target, cap);
  return (int)(g > min_blocks ? g : min_blocks);
}

// Every launcher returns the grid of the kernel that stores the mean's block partials.

template <typename T, int MODE, int NV, bool V4, bool AW = false>
int launch_wave(const void* z, const int64_t* y, int64_t N, int C, const Outs& o, hipStream_t s) {
  const void* k = reinterpret_cast<const void*>(&fwl_wave_rows<T, MODE, NV, V4, AW>);
  // fp32 register rows of >= 8000 bytes stream best from one block per CU (65536 x 2000: 184.8
  // against 196.9 us with two; 32768 x 2048: 95.7 against 97.7); 6000-7999 bytes gain nothing,
  // and 16-bit rows, bound by instruction issue, lose with fewer wavefronts
  const int64_t row_bytes = (int64_t)C * kElemBytes<T>;
  const int grid = wave_grid(N, row_bytes, resident_blocks(k), kElemBytes<T> == 4 && row_bytes >= 8000 ? 1 : 2);
  hipLaunchKernelGGL((fwl_wave_rows<T, MODE, NV, V4, AW>), dim3(grid), dim3(kBlock), 0, s, z, y, N, C, o);
  return grid;
}

// Whether line-aligned windows apply to a launch of the register-row kernel with `spare` unused
// 16-byte units per lane row (64*NV minus the row's units): contiguous rows (logits row stride C)
// of 16-byte multiples from 16-byte aligned logits and gradient that share their offset within a
// 128-byte line, with at least one row starting inside a line whose window fits (shift <= spare).
// Row starts repeat mod 128 every 8 rows.
bool windows_apply(const void* z, const void* g, int64_t N, int64_t row_bytes, int64_t ld_bytes, int spare) {
  const uintptr_t zp = reinterpret_cast<uintptr_t>(z), gp = reinterpret_cast<uintptr_t>(g);
  if (g == nullptr || ld_bytes != row_bytes || row_bytes % 16 != 0 || zp % 16 != 0 || gp % 16 != 0 ||
      (zp - gp) % 128 != 0)
    return false;
  for (int64_t r = 0; r < 8 && r < N; ++r) {
    const int a = (int)(((zp + (uintptr_t)(r * row_bytes)) >> 4) & 7);
    if (a > 0 && a <= spare) return true;
  }
  return false;
}

// register tier of a row of `units` 128-bit units per lane: NV = 1, 2, 3, 4, 5, 6 or 8
inline int wave_tier(int units) {
  return units <= 384 ? (units + 63) / 64 : 8;
}

template <typename T, int MODE, int NV>
int launch_wave_v4(const void* z, const int64_t* y, int64_t N, int C, bool aw, const Outs& o, hipStream_t s) {
  if constexpr (std::is_same<T, float>::value && MODE == kGrad) {
    if (aw) return launch_wave<T, MODE, NV, true, true>(z, y, N, C, o, s);
  }
  return launch_wave<T, MODE, NV, true>(z, y, N, C, o, s);
}

// register rows: NV units per lane, the smallest power of two that covers the row (E <= 32)
template <typename T, int MODE>
int dispatch_wave(const void* z, const int64_t* y, int64_t N, int C, bool v4, const Outs& o, const Params& p,
                  hipStream_t s) {
  if (v4) {
    // per-lane work grows with NV whatever the row length: tiers at every 64 units up to 6
    constexpr int U = kUnit<T, true>;
    const int units = (C + U - 1) / U;
    // line-aligned windows for the fp32 gradient rows whose window fits the row's own tier
    bool aw = false;
    if constexpr (std::is_same<T, float>::value && MODE == kGrad)
      aw = !p.no_window && windows_apply(z, o.grad, N, (int64_t)C * kElemBytes<T>, o.ld * kElemBytes<T>,
                                         kWave * wave_tier(units) - units);
    if (units <= 64) return launch_wave_v4<T, MODE, 1>(z, y, N, C, aw, o, s);
    if (units <= 128) return launch_wave_v4<T, MODE, 2>(z, y, N, C, aw, o, s);
    if (units <= 192) return launch_wave_v4<T, MODE, 3>(z, y, N, C, aw, o, s);
    if (units <= 256) return launch_wave_v4<T, MODE, 4>(z, y, N, C, aw, o, s);
    if constexpr (U == 4) {
      if (units <= 320) return launch_wave_v4<T, MODE, 5>(z, y, N, C, aw, o, s);
      if (units <= 384) return launch_wave_v4<T, MODE, 6>(z, y, N, C, aw, o, s);
      return launch_wave_v4<T, MODE, 8>(z, y, N, C, aw, o, s);
    }
    return 0;   // not reached: the host keeps 16-bit register rows within 256 units
  }
  if (C <= 64) return launch_wave<T, MODE, 1, false>(z, y, N, C, o, s);
  if (C <= 128) return launch_wave<T, MODE, 2, false>(z, y, N, C, o, s);
  if (C <= 256) return launch_wave<T, MODE, 4, false>(z, y, N, C, o, s);
  if (C <= 512) return launch_wave<T, MODE, 8, false>(z, y, N, C, o, s);
  return launch_wave<T, MODE, 16, false>(z, y, N, C, o, s);
}

template <typename T, int MODE, int L, int NV, bool V4>
int launch_seg(const void* z, const int64_t* y, int64_t N, int C, const Outs& o, hipStream_t s) {
  constexpr int R = kWave / L;
  const void* k = reinterpret_cast<const void*>(&fwl_seg_rows<T, MODE, L, NV, V4>);
  const int64_t groups = (N + R - 1) / R;
  // the wave grid over row groups (R rows each); a wavefront takes at most 64 / R groups
  const int resident = resident_blocks(k);
  const int cus = device_cus();
  const int64_t group_bytes = (int64_t)R * C * kElemBytes<T>;
  int per_cu = (int)((8000 + group_bytes - 1) / group_bytes);
  if (per_cu < 2) per_cu = 2;
  const int per_cu_resident = cus > 0 && resident > 0 ? resident / cus : 0;
  if (per_cu_resident > 0 && per_cu > per_cu_resident) per_cu = per_cu_resident;
  const int target = cus > 0 ? per_cu * cus : (resident > 0 ? resident : kMaxBlocksWave);
  const int64_t per_block = (int64_t)kWavesPerBlock * (kWave / R);
  const int64_t min_blocks = (groups + per_block - 1) / per_block;
  const int cap = (int)(min_blocks > kMaxBlocksWave ? min_blocks : kMaxBlocksWave);
  int64_t g = persistent_grid(groups, kWavesPerBlock, target, cap);
  if (g < min_blocks) g = min_blocks;
  hipLaunchKernelGGL((fwl_seg_rows<T, MODE, L, NV, V4>), dim3((int)g), dim3(kBlock), 0, s, z, y, N, C, o);
  return (int)g;
}

// short rows: segments of 16 or 32 lanes; returns 0 (nothing launched) when the row is too long
template <typename T, int MODE>
int dispatch_seg(const void* z, const int64_t* y, int64_t N, int C, bool v4, const Outs& o, hipStream_t s) {
  if constexpr (MODE == kCand) {
    return 0;
  } else {
    if (v4) {
      constexpr int U = kUnit<T, true>;
      const int units = C / U;
      if (units <= 16) return launch_seg<T, MODE, 16, 1, true>(z, y, N, C, o, s);
      if (units <= 32) return launch_seg<T, MODE, 16, 2, true>(z, y, N, C, o, s);
      if (units <= 64) return launch_seg<T, MODE, 32, 2, true>(z, y, N, C, o, s);
      return 0;
    }
    if (C <= 16) return launch_seg<T, MODE, 16, 1, false>(z, y, N, C, o, s);
    if (C <= 32) return launch_seg<T, MODE, 16, 2, false>(z, y, N, C, o, s);
    if (C <= 64) return launch_seg<T, MODE, 16, 4, false>(z, y, N, C, o, s);
    if (C <= 128) return launch_seg<T, MODE, 32, 4, false>(z, y, N, C, o, s);
    return 0;
  }
}

// The rows a streaming launch deferred (their lists overflowed): fwl_overflow_rows right after it,
// its block partials after the streaming kernel's `grid1`.  Nothing to launch without the
// workspace's overflow records (the streaming kernels then solve such rows themselves).
template <typename T, int MODE, bool V4>
int launch_overflow(const void* z, const int64_t* y, int64_t N, int C, Outs o, int grid1, hipStream_t s) {
  if (o.ovf_lo == nullptr) return 0;
  if (o.partials != nullptr) o.partials += grid1;
  const void* k = reinterpret_cast<const void*>(&fwl_overflow_rows<T, MODE, V4>);
  const int grid = persistent_grid(N, 1, resident_blocks(k), kMaxBlocksRow);
  hipLaunchKernelGGL((fwl_overflow_rows<T, MODE, V4>), dim3(grid), dim3(kBlock), 0, s, z, y, N, C, o);
  return grid;
}

// (OV4: the access width of the overflow kernel after the stream, which reads rows from their
// own start: 16-bit rows that the stream read through windows take 16-bit accesses there)
template <typename T, int MODE, bool V4, bool BIG = false, bool OV4 = V4>
int launch_block(const void* z, const int64_t* y, int64_t N, int C, const Outs& o, hipStream_t s) {
  const void* k = reinterpret_cast<const void*>(&fwl_block_rows<T, MODE, V4, BIG>);
  const int grid = persistent_grid(N, 1, resident_blocks(k), kMaxBlocksRow);
  hipLaunchKernelGGL((fwl_block_rows<T, MODE, V4, BIG>), dim3(grid), dim3(kBlock), 0, s, z, y, N, C, o);
  return grid + launch_overflow<T, MODE, OV4>(z, y, N, C, o, grid, s);
}

template <typename T, int MODE, bool V4, bool OV4 = V4, bool LONG = false>
int launch_wave_stream(const void* z, const int64_t* y, int64_t N, int C, const Outs& o, hipStream_t s) {
  const void* k = reinterpret_cast<const void*>(&fwl_wave_stream_rows<T, MODE, V4, LONG>);
  const int grid = wave_grid(N, (int64_t)C * kElemBytes<T>, resident_blocks(k));
  hipLaunchKernelGGL((fwl_wave_stream_rows<T, MODE, V4, LONG>), dim3(grid), dim3(kBlock), 0, s, z, y, N, C, o);
  return grid + launch_overflow<T, MODE, OV4>(z, y, N, C, o, grid, s);
}

size_t mean_ws_bytes(int64_t N);
size_t ovf_ws_bytes(int64_t N);
size_t two_pass_bytes(int64_t N);
// The fused op in two passes: the candidate-list kernel (support indices of rows whose lists kept
// them, at most kTwoPassCap per row, in the workspace after the mean's part), then the write
// pass: fwl_write_flat and fwl_scatter_support for rows of whole 128-bit units, else
// fwl_fill_zero and fwl_scatter_support.
template <typename T, bool V4>
int launch_two_pass(const void* z, const int64_t* y, int64_t N, int C, const Outs& o, void* ws, size_t ws_bytes,
                    hipStream_t s) {
  char* base = static_cast<char*>(ws) + mean_ws_bytes(N) + ovf_ws_bytes(N);
  const size_t L = (size_t)N * kTwoPassCap;
  Outs o1 = o;
  o1.cval = nullptr;   // indices only
  o1.cidx = reinterpret_cast<int32_t*>(base);
  o1.ccnt = reinterpret_cast<int32_t*>(base + sizeof(int32_t) * L);
  float* Hs = reinterpret_cast<float*>(base + sizeof(int32_t) * L + sizeof(int32_t) * (size_t)N);
  o1.cstride = kTwoPassCap;
  o1.ccap = kTwoPassCap;
  o1.mark_unlisted = 1;
  if (o1.H == nullptr) o1.H = Hs;
  o1.grad = nullptr;
  // The read pass streams one row per wavefront when there are rows for kTwoPassWaveRowsPerCU
  // wavefronts per CU (8192 x 32000: 178 us against 206 us with one block per row), else one row
  // per block (520 x 128256: 181 us with one row per wavefront, 119 us per block), both with long
  // lists.
  // 16-bit rows without 128-bit units (odd lengths or strides) are read one row per wavefront
  // through windows from the 4-byte boundary below each row (win_shift), their overflow solve with
  // 16-bit elements; read one row per block they stay on 16-bit elements (windows measured slower
  // there at N(0, 0.01^2): 600 x 65537 bf16 166 against 78 us)
  constexpr bool kWin = !V4 && kElemBytes<T> == 2;
  int grid;
  if (N >= kTwoPassWaveRowsPerCU * (int64_t)device_cus())
    grid = launch_wave_stream<T, kCand, V4 || kWin, V4, true>(z, y, N, C, o1, s);
  else
    grid = launch_block<T, kCand, V4, true>(z, y, N, C, o1, s);
  const int64_t row_bytes = (int64_t)C * kElemBytes<T>;
  if (V4 && row_bytes % 16 == 0) {
    const int64_t wb = (N * row_bytes + kWriteBytes - 1) / kWriteBytes;
    hipLaunchKernelGGL((fwl_write_flat<T>), dim3((unsigned)wb), dim3(kBlock), 0, s, z, o.ld, y, o1.H, o1.ccnt, N, C,
                       o.scale, o.scale_f, o.grad);
    hipLaunchKernelGGL((fwl_scatter_support<T, V4>), dim3(blocks_wave(N)), dim3(kBlock), 0, s, z, o.ld, y, o1.H,
                       o1.ccnt, o1.cidx, N, C, o.scale, o.scale_f, o.grad, false, kLongDone);
    return grid;
  }
  const int64_t bytes = N * (int64_t)C * kElemBytes<T>;
  const int64_t fill_blocks = (bytes + kFillBytes - 1) / kFillBytes;
  // rows whose support outgrew the lists are written whole by the scatter kernel, and the fill
  // leaves them alone, where rows are whole dwords and at least a fill block long
  const bool dense = row_bytes % 4 == 0 && row_bytes >= kFillBytes;
  hipLaunchKernelGGL(fwl_fill_zero, dim3((unsigned)fill_blocks), dim3(kBlock), 0, s, o.grad, bytes, row_bytes,
                     dense ? o1.ccnt : nullptr);
  hipLaunchKernelGGL((fwl_scatter_support<T, V4>), dim3(blocks_wave(N)), dim3(kBlock), 0, s, z, o.ld, y, o1.H, o1.ccnt,
                     o1.cidx, N, C, o.scale, o.scale_f, o.grad, (bytes & 3) != 0, dense ? kLongDense : kLongScan);
  return grid;
}


// Split rows: chunks of whole streaming rounds (`round` elements; 16-byte aligned whenever the
// row is), about kSplitTargetItems (row, chunk) items in all, at most kSplitMaxChunks per row.
struct SplitPlan {
  int nch;   // chunks per row
  int CH;    // elements per chunk (the last one may be shorter)
};

// chunks per row before rounding the chunk length up to whole rounds: an upper bound of
// split_plan(N, C, round).nch for every round >= kSplitMinChunk (sizes the workspace)
int64_t split_chunks_bound(int64_t N, int64_t C, int64_t round) {
  int64_t nch = (kSplitTargetItems + N - 1) / (N > 0 ? N : 1);
  const int64_t by_c = (C + round - 1) / round;
  if (nch > kSplitMaxChunks) nch = kSplitMaxChunks;
  if (nch > by_c) nch = by_c;
  return nch < 1 ? 1 : nch;
}

SplitPlan split_plan(int64_t N, int64_t C, int64_t round) {
  const int64_t nch = split_chunks_bound(N, C, round);
  int64_t CH = (C + nch - 1) / nch;
  CH = (CH + round - 1) / round * round;
  return {(int)((C + CH - 1) / CH), (int)CH};
}

// whether rows of this shape (elements of `elem` bytes) take the split kernels under dispatch
// switch `path`; elem = 4 answers for every element type (the workspace size)
bool split_rows(int64_t N, int64_t C, int64_t elem, int path) {
  return N >= 1 && N <= kSplitMaxRows && C >= 1 && (path == 7 || (path == 0 && C * elem >= kSplitMinBytes));
}

// fp64 partial sums of the mean: one per block of the two largest grids a forward launches for N
// rows (a streaming kernel, then fwl_overflow_rows)
int64_t partial_slots(int64_t N) {
  const int64_t wave_max = (N + (int64_t)kWavesPerBlock * kRowsPerWave - 1) / ((int64_t)kWavesPerBlock * kRowsPerWave);
  int64_t b = kMaxBlocksRow > kMaxBlocksWave ? kMaxBlocksRow : kMaxBlocksWave;
  if (b < kSplitMaxRows) b = kSplitMaxRows;
  return 2 * (wave_max > b ? wave_max : b);
}


inline size_t ws_round(size_t b) { return (b + kWsAlign - 1) / kWsAlign * kWsAlign; }

// the mean's part of the workspace: the block partials
size_t mean_ws_bytes(int64_t N) { return ws_round(sizeof(double) * (size_t)partial_slots(N)); }

// the overflow records of the streaming kernels: a lower bound and the maximum per row
size_t ovf_ws_bytes(int64_t N) { return ws_round(2 * sizeof(float) * (size_t)(N > 0 ? N : 0)); }

// Whether the fused op may run in two passes (the long-row block path) under switch `path`.
// Measured on MI355X against one pass (fp32): 8192 x 32000 423 -> 400 us, 2048 x 131072 378 ->
// 357 us, 520 x 128256 132 -> 118 us, 400 x 50257 50.5 -> 46.8 us; but 256 x 128256 67 -> 79 us.
// With the fill-and-scatter write pass, large fp32 batches of shorter rows gain too (256 MB of
// logits): 8192 x 8192 102.0 -> 95.6 us, 5592 x 12000 113.5 -> 96.6, 4096 x 16384 106.2 -> 93.5,
// 2796 x 24000 119.7 -> 106.8; with the current read pass also from 128 MB (4096 x 10000 78.4 ->
// 69.8 us, 2560 x 16384 80.2 -> 75.2, 1700 x 24000 79.7 -> 74.4, 2048 x 16384 63.2 -> 59.9;
// 3000 x 10000 even), below it one pass wins (16-64 MB: 18-36 us against 22-43).  bf16 (against one row per block): 2048 x 131072 218 -> 190 us; with the
// read pass's sparse and two-entry rounds, rows of 32000-50000 elements gain once the read pass
// takes one row per wavefront (8192 x 32000 242 -> 203 us, 4096 x 32000 130 -> 114, 2048 x 40000
// 88 -> 77, 4096 x 50000 199 -> 155) but not below that (1024 x 32000 46 -> 56).  Automatic
// dispatch: fp32 rows of >= 32000 elements, >= 384 of them, or of >= 8192 elements in batches of
// >= 32M elements; 16-bit rows of >= 65536 elements, >= 512 of them, or of >= 32000 elements,
// kTwoPassWaveRowsPerCU of them per CU.  Forced paths 2 and 3 always (their tests exercise both
// passes in every element type).
constexpr int64_t kTwoPassMinC = 32000;
constexpr int64_t kTwoPassMinRows = 384;
constexpr int64_t kTwoPassMinCBig = 8192;
constexpr int64_t kTwoPassMinElemsBig = (int64_t)32 << 20;
constexpr int64_t kTwoPassMinC16 = 65536;
constexpr int64_t kTwoPassMinRows16 = 512;
// 16-bit rows of 28000-31999 elements, at twice kTwoPassWaveRowsPerCU rows per CU: 8192 x 28000
// 193.1 -> 183.8 us, 8192 x 30000 211.7 -> 192.7, 4096 x 28000 even; 24000 elements lose
// (4096 x 24000 90.8 -> 97.0, 8192 x 24000 165.5 -> 170.6)
constexpr int64_t kTwoPassMinC16Many = 28000;
bool two_pass_rows(int64_t N, int64_t C, int64_t elem, int path) {
  if (path == 2 || path == 3) return true;
  if (path != 0) return false;
  if (elem == 4)
    return (C >= kTwoPassMinC && N >= kTwoPassMinRows) || (C >= kTwoPassMinCBig && N * C >= kTwoPassMinElemsBig);
  const int64_t w = kTwoPassWaveRowsPerCU * (int64_t)device_cus();
  return (C >= kTwoPassMinC16 && N >= kTwoPassMinRows16) || (C >= kTwoPassMinC && N >= w) ||
         (C >= kTwoPassMinC16Many && N >= 2 * w);
}

// 16-bit rows beyond kMaxStreamC stream faster on one wavefront each than on one block each once
// there are enough rows (bf16, one wavefront per row against one block per row): 5592 x 12000
// 65.7 us against 98.1, 4096 x 16384 61.7 against 79.7, 1198 x 28000 43.1 against 50.3, 1024 x
// 32000 40.9 against 46.4, 1024 x 50000 55.7 against 62.5; below about 1024 rows one block per
// row wins (512 x 32000: 38.7 against 31.9).  From 65536 elements the two passes take them.
// Rows without 128-bit units (16-bit loads) stream up to the length measured before.
constexpr int kMaxStreamC16 = 65535;
constexpr int kMaxStreamC16V1 = 28672;
constexpr int64_t kStreamMinRows16 = 1024;

// the two passes' scratch: cut candidate lists (values, indices), kappa and H per row
size_t two_pass_bytes(int64_t N) {
  return (size_t)N * (kTwoPassCap * sizeof(int32_t) + sizeof(int32_t) + sizeof(float));
}


size_t split_scratch_bytes(int64_t N, int64_t C) {
  const int64_t items = N * split_chunks_bound(N, C, kSplitMinChunk);
  return (size_t)items * (sizeof(double) + sizeof(int) + sizeof(float) + (size_t)kSplitCap * (sizeof(float) + sizeof(int)));
}

size_t workspace_bytes(int64_t N, int64_t C, int path) {
  if (N < 0) N = 0;
  // the fp64 partials of the mean, the overflow records, then the larger of the split rows' and
  // the two passes' scratch
  size_t extra = 0;
  if (split_rows(N, C, 4, path)) extra = split_scratch_bytes(N, C);
  // (16-bit rows without 128-bit units take two passes from kTwoPassMinCWin16 elements at
  // kTwoPassWaveRowsPerCU rows per CU; without a device, per 256 CUs)
  const int cus = device_cus();
  const bool win16 = C >= kTwoPassMinCWin16 && N >= kTwoPassWaveRowsPerCU * (int64_t)(cus > 0 ? cus : 256);
  if ((two_pass_rows(N, C, 4, path) || (path == 0 && win16)) && two_pass_bytes(N) > extra) extra = two_pass_bytes(N);
  return mean_ws_bytes(N) + ovf_ws_bytes(N) + extra;
}

template <typename T, int MODE, bool V4>
int launch_split(const void* z, const int64_t* y, int64_t N, int C, const Outs& o, void* ws, hipStream_t s) {
  constexpr int kRound = kWave * kWavesPerBlock * Round<T, V4>::kSlots;
  static_assert(kRound >= kSplitMinChunk, "the workspace bound assumes rounds of >= kSplitMinChunk elements");
  const SplitPlan pl = split_plan(N, C, kRound);
  const int64_t items = N * split_chunks_bound(N, C, kSplitMinChunk);   // the workspace layout
  char* base = static_cast<char*>(ws) + mean_ws_bytes(N) + ovf_ws_bytes(N);
  SplitScratch sc;
  sc.tau = reinterpret_cast<double*>(base);
  sc.count = reinterpret_cast<int*>(base + sizeof(double) * items);
  sc.mx = reinterpret_cast<float*>(base + (sizeof(double) + sizeof(int)) * items);
  sc.val = reinterpret_cast<float*>(base + (sizeof(double) + sizeof(int) + sizeof(float)) * items);
  sc.idx = reinterpret_cast<int*>(base + (sizeof(double) + sizeof(int) + sizeof(float) + sizeof(float) * kSplitCap) * items);
  const void* ka = reinterpret_cast<const void*>(&fwl_split_chunks<T, MODE, V4>);
  const int ga = persistent_grid(N * (int64_t)pl.nch, 1, resident_blocks(ka), kMaxBlocksRow);
  hipLaunchKernelGGL((fwl_split_chunks<T, MODE, V4>), dim3(ga), dim3(kBlock), 0, s, z, N, C, pl.CH, pl.nch, o, sc);
  const int gb = (int)N;   // N <= kSplitMaxRows
  hipLaunchKernelGGL((fwl_split_finish<T, MODE, V4>), dim3(gb), dim3(kBlock), 0, s, z, y, N, C, pl.nch, o, sc);
  return gb;
}

// rows are addressed through buffer resources with 32-bit byte ranges and offsets (one round
// past the row end included), hence the bound on C

// Shared forward driver; `out_v4_ok` says whether the mode's dense output allows 128-bit access.
// ld is the logits' row stride in elements (>= C).  The mean's block partials go to the start of
// the workspace and fwl_mean_finish adds them after the rows.
template <typename T, int MODE>
int forward(const void* z, int64_t ld, const int64_t* y, int64_t N, int64_t C64, double scale, double reduce_div,
            Outs o, bool out_v4_ok, void* ws, size_t ws_bytes, const Params& p, hipStream_t s) {
  if (bad_shape(N, C64) || ld < C64 || ld > kMaxC || (N > 0 && (z == nullptr || y == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(z, kElemBytes<T>) || !aligned(y, 8)) return FWL_ERR_ALIGNMENT;
  const int C = (int)C64;
  // every row's byte range must fit the buffer resources' 32-bit offsets (checked on C by
  // bad_shape); rows further apart than that are addressed from their own base
  o.scale = scale;
  o.reduce_div = reduce_div;
  o.scale_f = (float)scale;
  o.ld = ld;
  o.cap = p.cap;
  o.force_generic = p.path == 3 || p.path == 5;
  o.partials = nullptr;
  o.ovf_lo = o.ovf_mx = nullptr;
  const bool ws_ok = ws != nullptr && aligned(ws, 8);
  if (o.mean != nullptr) {
    if (!ws_ok || ws_bytes < mean_ws_bytes(N)) return FWL_ERR_WORKSPACE;
    o.partials = static_cast<double*>(ws);
  }
  const size_t ws_head = mean_ws_bytes(N) + ovf_ws_bytes(N);   // where the long rows' scratch starts
  if (ws_ok && ws_bytes >= ws_head) {
    o.ovf_lo = reinterpret_cast<float*>(static_cast<char*>(ws) + mean_ws_bytes(N));
    o.ovf_mx = o.ovf_lo + N;
  }
  if (N == 0) {
    if (o.mean != nullptr) hipLaunchKernelGGL(fwl_empty_mean, dim3(1), dim3(1), 0, s, o.mean, reduce_div);
    return launch_status();
  }
  // 128-bit units: rows of 16-byte multiples from a 16-byte aligned start; fp32 rows of any length
  // and 16-bit rows of even length also take them (the buffer range check is per dword: a last unit
  // that runs past the row loads zeros there and stores nothing there; unaligned starts are
  // supported)
  const bool aligned_rows = (C % kUnit<T, true>) == 0 && (ld % kUnit<T, true>) == 0 && aligned(z, 16) && out_v4_ok;
  // 16-bit rows of even length start on 4-byte boundaries: every dword holds two elements of one
  // row, so the per-dword range check serves them as it serves fp32 rows of any length (bf16,
  // against 16-bit accesses: 1002 elements 3.73 -> 4.44 TB/s, 8194 3.58 -> 4.10, 50002 2.29 ->
  // 3.48; rows of up to 256 elements keep the 16-bit accesses, which fill more lanes: 130
  // elements 1.20 against 1.03)
  const bool even16 = kElemBytes<T> == 2 && MODE == kGrad && C % 2 == 0 && ld % 2 == 0 && C > 256 && aligned(z, 4) &&
                      aligned(o.grad, 4);
  const bool v4 = aligned_rows || (std::is_same<T, float>::value && MODE != kMask) || even16;
  int path = p.path == 8 ? 1 : p.path;
  // measured on MI355X: registers win up to 2048 for 128-bit rows, up to 1024 for rows accessed
  // one element at a time; one streaming wavefront per row up to 8192; one block per row beyond
  const int max_wave_c = v4 ? kMaxWaveC : kMaxWaveC1;
  const size_t ws_have = ws_ok ? ws_bytes : 0;
  int grid = 0;
  // few long rows: chunks of every row on their own blocks (needs the scratch of the workspace)
  if (path == 0 && split_rows(N, C, kElemBytes<T>, 0)) path = 7;
  if (path == 7) {
    if (split_rows(N, C, kElemBytes<T>, 7) && ws_have >= ws_head + split_scratch_bytes(N, C)) {
      grid = v4 ? launch_split<T, MODE, true>(z, y, N, C, o, ws, s) : launch_split<T, MODE, false>(z, y, N, C, o, ws, s);
      path = -1;
    } else {
      path = 2;
    }
  }
  const bool two_pass_ok = MODE == kGrad && aligned(o.grad, 4) && ws_have >= ws_head + two_pass_bytes(N);
  // 16-bit rows without 128-bit units (odd lengths or strides), long and many: the two-pass op,
  // whose read pass takes them through windows with 128-bit loads (bf16 2048 x 50257: 188 -> 100 us,
  // 8192 x 32001: 414 -> 238; the same at N(0, 0.01^2); fewer rows read one block per row, which
  // lost at N(0, 0.01^2): 512 x 50257 140 against 70).  From kTwoPassMinCWin16 elements against
  // the one-pass stream with 16-bit loads: 2048 x 12001 47.3 -> 41.1 us, 4095 x 16385 83.1 -> 72.8,
  // 2048 x 24001 69.9 -> 55.1, 8191 x 12001 115.3 -> 112.3; at 8193 elements it is even or loses.
  const bool win16 = kElemBytes<T> == 2 && !v4 && C >= kTwoPassMinCWin16 &&
                     N >= kTwoPassWaveRowsPerCU * (int64_t)device_cus();
  if (path == 0 && !aligned_rows && C <= 128) path = 6;   // short unaligned rows: 32-bit segments
  if (path == 0) {
    const bool two_pass = two_pass_ok && (two_pass_rows(N, C, kElemBytes<T>, 0) || win16);
    const bool stream = C <= kMaxStreamC ||
                        (kElemBytes<T> == 2 && C <= (v4 ? kMaxStreamC16 : kMaxStreamC16V1) && N >= kStreamMinRows16);
    path = C <= max_wave_c ? 6 : (two_pass ? 2 : (stream ? 4 : 2));
  }
  if ((path == 1 || path == 6) && C > max_wave_c) path = 4;
  if (path == 6) {
    grid = dispatch_seg<T, MODE>(z, y, N, C, aligned_rows, o, s);
    if (grid > 0) path = -1;
  }
  if (path == 1 || path == 6) {
    grid = dispatch_wave<T, MODE>(z, y, N, C, v4, o, p, s);
  } else if (path == 4 || path == 5) {
    grid = v4 ? launch_wave_stream<T, MODE, true>(z, y, N, C, o, s) : launch_wave_stream<T, MODE, false>(z, y, N, C, o, s);
  } else if (path >= 0) {
    if (two_pass_ok && (two_pass_rows(N, C, kElemBytes<T>, p.path) || (p.path == 0 && win16))) {
      grid = v4 ? launch_two_pass<T, true>(z, y, N, C, o, ws, ws_have, s)
                : launch_two_pass<T, false>(z, y, N, C, o, ws, ws_have, s);
    } else {
      grid = v4 ? launch_block<T, MODE, true>(z, y, N, C, o, s) : launch_block<T, MODE, false>(z, y, N, C, o, s);
    }
  }
  if (o.mean != nullptr)
    hipLaunchKernelGGL(fwl_mean_finish, dim3(1), dim3(kWave), 0, s, o.partials, (unsigned)grid, reduce_div, o.mean);
  return launch_status();
}

template <typename T>
int scale_grad(void* grad, const float* grad_output, int64_t go_stride, int64_t N, int64_t C, hipStream_t stream) {
  if (bad_shape(N, C) || go_stride < 0 || (N > 0 && (grad == nullptr || grad_output == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(grad, kElemBytes<T>) || !aligned(grad_output, 4)) return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  const int Ci = (int)C;
  if ((C % kUnit<T, true>) == 0 && aligned(grad, 16))
    hipLaunchKernelGGL((fwl_scale_rows<T, true>), dim3(blocks_wave(N)), dim3(kBlock), 0, stream, grad, grad_output,
                       go_stride, N, Ci);
  else
    hipLaunchKernelGGL((fwl_scale_rows<T, false>), dim3(blocks_wave(N)), dim3(kBlock), 0, stream, grad, grad_output,
                       go_stride, N, Ci);
  return launch_status();
}

// the fused op for any element type (fwl_forward_backward_ex and the entry points over it)
int fused_forward(int dtype, const void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C,
                  double scale, double reduce_div, float* H, float* losses, double* losses64, float* mean_loss,
                  int32_t* kappa, void* grad, void* workspace, size_t workspace_bytes, const Params& p,
                  hipStream_t stream) {
  if (N > 0 && grad == nullptr) return FWL_ERR_INVALID_ARG;
  Outs o = {};
  o.H = H;
  o.loss = losses;
  o.loss64 = losses64;
  o.mean = mean_loss;
  o.kappa = kappa;
  o.grad = grad;
  switch (dtype) {
    case FWL_FLOAT32:
      if (!aligned(grad, 4)) return FWL_ERR_ALIGNMENT;
      return forward<float, kGrad>(logits, ld, targets, N, C, scale, reduce_div, o, aligned(grad, 16), workspace,
                                   workspace_bytes, p, stream);
    case FWL_BFLOAT16:
      if (!aligned(grad, 2)) return FWL_ERR_ALIGNMENT;
      return forward<bf16_t, kGrad>(logits, ld, targets, N, C, scale, reduce_div, o, aligned(grad, 16), workspace,
                                    workspace_bytes, p, stream);
    case FWL_FLOAT16:
      if (!aligned(grad, 2)) return FWL_ERR_ALIGNMENT;
      return forward<f16_t, kGrad>(logits, ld, targets, N, C, scale, reduce_div, o, aligned(grad, 16), workspace,
                                   workspace_bytes, p, stream);
    default:
      return FWL_ERR_INVALID_ARG;
  }
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// The workspace of fwl_forward_backward_noalloc: one array per device, in the code object, so that
// the entry point allocates nothing.  In host code `scratch` is only a host-side stand-in for the
// symbol; its device address (one per device) comes from hipGetSymbolAddress and is the only
// address passed to kernels.  The library keeps no state in a workspace between calls, so nothing
// in it needs clearing; calls that overlap on one device share it and race.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

// the device address of `scratch` on the current device (looked up once per device)
int scratch_address(void** out) {
  static std::mutex mu;
  static std::map<int, void*> addr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FWL_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(mu);
  auto it = addr.find(dev);
  if (it == addr.end()) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return FWL_ERR_DEVICE;
    it = addr.emplace(dev, ptr).first;
  }
  *out = it->second;
  return FWL_OK;
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// C ABI

extern "C" {

const char* fwl_status_string(int status) {
  switch (status) {
    case FWL_OK: return "ok";
    case FWL_ERR_INVALID_ARG: return "invalid argument (null pointer, N < 0, C < 1, C too large, ld < C, or an option out of range)";
    case FWL_ERR_WORKSPACE: return "workspace missing, misaligned or smaller than fwl_workspace_bytes(N, C)";
    case FWL_ERR_ALIGNMENT: return "misaligned pointer (logits/grad need their element size, targets 8 bytes)";
    case FWL_ERR_LAUNCH: return "kernel launch failed (is the current device a gfx950?)";
    case FWL_ERR_DEVICE: return "no usable device";
    default: return "unknown fwloss status";
  }
}

size_t fwl_workspace_bytes(int64_t N, int64_t C) { return workspace_bytes(N, C, default_params().path); }

size_t fwl_workspace_bytes_ex(int64_t N, int64_t C, const fwl_options* options) {
  Params p;
  if (!call_params(options, p)) return 0;
  return workspace_bytes(N, C, p.path);
}

int fwl_forward_backward_ex(int dtype, const void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C,
                            double scale, double reduce_div, float* H, float* losses, double* losses64,
                            float* mean_loss, int32_t* kappa, void* grad, void* workspace, size_t workspace_bytes,
                            const fwl_options* options, hipStream_t stream) {
  Params p;
  if (!call_params(options, p)) return FWL_ERR_INVALID_ARG;
  return fused_forward(dtype, logits, ld, targets, N, C, scale, reduce_div, H, losses, losses64, mean_loss, kappa,
                       grad, workspace, workspace_bytes, p, stream);
}

size_t fwl_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int fwl_forward_backward_noalloc(int dtype, const void* logits, int64_t ld, const int64_t* targets, int64_t N,
                                 int64_t C, double scale, double reduce_div, float* H, float* losses,
                                 double* losses64, float* mean_loss, int32_t* kappa, void* grad,
                                 const fwl_options* options, hipStream_t stream) {
  Params p;
  if (!call_params(options, p)) return FWL_ERR_INVALID_ARG;
  if (bad_shape(N, C)) return FWL_ERR_INVALID_ARG;
  // every part of the workspace this call would use must fit the static scratch
  if (workspace_bytes(N, C, p.path) > kNoAllocScratchBytes) return FWL_ERR_WORKSPACE;
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != FWL_OK) return rc;
  return fused_forward(dtype, logits, ld, targets, N, C, scale, reduce_div, H, losses, losses64, mean_loss, kappa,
                       grad, ws, kNoAllocScratchBytes, p, stream);
}

int fwl_forward_backward(const float* logits, const int64_t* targets, int64_t N, int64_t C,
                         double scale, double reduce_div, float* H, float* losses,
                         float* mean_loss, int32_t* kappa, float* grad, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  return fused_forward(FWL_FLOAT32, logits, C, targets, N, C, scale, reduce_div, H, losses, nullptr, mean_loss, kappa,
                       grad, workspace, workspace_bytes, default_params(), stream);
}

int fwl_forward_backward_typed(int dtype, const void* logits, const int64_t* targets, int64_t N, int64_t C,
                               double scale, double reduce_div, float* H, float* losses, float* mean_loss,
                               int32_t* kappa, void* grad, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  return fused_forward(dtype, logits, C, targets, N, C, scale, reduce_div, H, losses, nullptr, mean_loss, kappa, grad,
                       workspace, workspace_bytes, default_params(), stream);
}

int fwl_forward_small(const float* logits, const int64_t* targets, int64_t N, int64_t C,
                      float* H, float* losses, float* mean_loss, int32_t* kappa,
                      uint8_t* selected, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
  if (N > 0 && selected == nullptr) return FWL_ERR_INVALID_ARG;
  Outs o = {};
  o.H = H;
  o.loss = losses;
  o.mean = mean_loss;
  o.kappa = kappa;
  o.mask = selected;
  return forward<float, kMask>(logits, C, targets, N, C, N > 0 ? 1.0 / (double)N : 1.0, (double)N, o,
                               aligned(selected, 4), workspace, workspace_bytes, default_params(), stream);
}

int fwl_forward_large(const float* logits, const int64_t* targets, int64_t N, int64_t C,
                      float* H, float* losses, float* mean_loss, int32_t* kappa,
                      float* cand_values, int32_t* cand_indices, int32_t* cand_counts,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (N > 0 && (cand_values == nullptr || cand_indices == nullptr || cand_counts == nullptr))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(cand_values, 4) || !aligned(cand_indices, 4) || !aligned(cand_counts, 4))
    return FWL_ERR_ALIGNMENT;
  Outs o = {};
  o.H = H;
  o.loss = losses;
  o.mean = mean_loss;
  o.kappa = kappa;
  o.cval = cand_values;
  o.cidx = cand_indices;
  o.ccnt = cand_counts;
  o.cstride = (int)(C > 0 && C <= kMaxC ? C : 0);   // whole rows (checked again by forward)
  o.ccap = o.cstride;
  return forward<float, kCand>(logits, C, targets, N, C, N > 0 ? 1.0 / (double)N : 1.0, (double)N, o, true,
                               workspace, workspace_bytes, default_params(), stream);
}

int fwl_backward_small(const int64_t* targets, const uint8_t* selected, const int32_t* kappa,
                       int64_t N, int64_t C, float* grad, hipStream_t stream) {
  if (bad_shape(N, C) || (N > 0 && (targets == nullptr || selected == nullptr || kappa == nullptr ||
                                    grad == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(targets, 8) || !aligned(kappa, 4) || !aligned(grad, 4)) return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  const double scale = 1.0 / (double)N;
  const bool v4 = (C % 4) == 0 && aligned(selected, 4) && aligned(grad, 16);
  const int Ci = (int)C;
  // at most 64 rows per wavefront (the labels and kappas of its rows are gathered once)
  if (v4) {
    const int grid = wave_grid(N, 5 * C, resident_blocks(reinterpret_cast<const void*>(&fwl_mask_to_grad<true>)));
    hipLaunchKernelGGL((fwl_mask_to_grad<true>), dim3(grid), dim3(kBlock), 0, stream, targets, selected, kappa, N,
                       Ci, scale, (float)scale, grad);
  } else {
    const int grid = wave_grid(N, 5 * C, resident_blocks(reinterpret_cast<const void*>(&fwl_mask_to_grad<false>)));
    hipLaunchKernelGGL((fwl_mask_to_grad<false>), dim3(grid), dim3(kBlock), 0, stream, targets, selected, kappa, N,
                       Ci, scale, (float)scale, grad);
  }
  return launch_status();
}

int fwl_backward_large(const float* logits, const int64_t* targets, const float* H,
                       const int32_t* kappa, const float* cand_values,
                       const int32_t* cand_indices, const int32_t* cand_counts, int64_t N,
                       int64_t C, float* grad, hipStream_t stream) {
  if (bad_shape(N, C) || (N > 0 && (logits == nullptr || targets == nullptr || H == nullptr ||
                                    kappa == nullptr || cand_values == nullptr ||
                                    cand_indices == nullptr || cand_counts == nullptr || grad == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(logits, 4) || !aligned(targets, 8) || !aligned(grad, 4)) return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  const double scale = 1.0 / (double)N;
  const bool v4 = (C % 4) == 0 && aligned(grad, 16);
  const int Ci = (int)C;
  if (v4)
    hipLaunchKernelGGL((fwl_cand_to_grad<true>), dim3(blocks_row(N)), dim3(kBlock), 0, stream, logits,
                       targets, H, kappa, cand_values, cand_indices, cand_counts, N, Ci, scale,
                       (float)scale, grad);
  else
    hipLaunchKernelGGL((fwl_cand_to_grad<false>), dim3(blocks_row(N)), dim3(kBlock), 0, stream, logits,
                       targets, H, kappa, cand_values, cand_indices, cand_counts, N, Ci, scale,
                       (float)scale, grad);
  return launch_status();
}

int fwl_scale_grad(float* grad, const float* grad_output, int64_t go_stride, int64_t N, int64_t C,
                   hipStream_t stream) {
  return scale_grad<float>(grad, grad_output, go_stride, N, C, stream);
}

int fwl_scale_grad_typed(int dtype, void* grad, const float* grad_output, int64_t go_stride, int64_t N, int64_t C,
                         hipStream_t stream) {
  switch (dtype) {
    case FWL_FLOAT32: return scale_grad<float>(grad, grad_output, go_stride, N, C, stream);
    case FWL_BFLOAT16: return scale_grad<bf16_t>(grad, grad_output, go_stride, N, C, stream);
    case FWL_FLOAT16: return scale_grad<f16_t>(grad, grad_output, go_stride, N, C, stream);
    default: return FWL_ERR_INVALID_ARG;
  }
}

int fwl_set_params(int path, int cand_cap) {
  if (path < 0 || path > 8 || cand_cap < kWave || cand_cap > kCapMax) return FWL_ERR_INVALID_ARG;
  g_path.store(path, std::memory_order_relaxed);
  g_cap.store(cand_cap, std::memory_order_relaxed);
  return FWL_OK;
}

int fwl_get_params(int* path, int* cand_cap) {
  if (path) *path = g_path.load(std::memory_order_relaxed);
  if (cand_cap) *cand_cap = g_cap.load(std::memory_order_relaxed);
  return FWL_OK;
}


}  // extern "C"
