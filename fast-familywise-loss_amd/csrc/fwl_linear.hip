// fwl_linear.hip -- the linear layer that produces the logits (an LM head) fused with the FW loss,
// for libfwloss.so (the fwl_linear_* entry points of include/fwloss.h).  No counterpart in the
// reference, whose losses take materialised logits.
//
// Compile with -Xclang -target-feature -Xclang -packed-fp32-ops (see fwloss_build.py).
#include "fwl_common.h"

namespace {

// ------------------------------------------------------------------------------------------------
// The linear layer that produces the logits, fused with the loss: logits = hidden @ weight^T
// arrive one vocabulary chunk at a time ([N, Vc] for columns v0 .. v0 + Vc - 1), and no [N, V]
// logits tensor ever exists.  Per row a state in device memory carries, from chunk to chunk, the
// running maximum m, a lower bound t <= tau (max(m - 1, H(list)) rounded down) and the list of
// every entry seen so far that is > t (value and column).  Every support entry of the full row is
// > t at every step, so after the last chunk the list holds the support and the row maximum, and
// the threshold is resolved on it exactly as for a materialised row.  Rows whose list outgrows
// kLinCap entries above the bound (or a chunk's kLinLds), and rows without a finite maximum, are
// flagged; the caller runs them through the materialised path.
//
// The gradient of the loss with respect to the logits has kappa + 1 non-zeros per row, so the
// backward needs no GEMM: dhidden[n] = sum_j g_nj weight[j] (a gather of kappa + 1 weight rows)
// and dweight[j] = sum_n g_nj hidden[n] (one pass over (column, row) entries sorted by column).

constexpr int kLinCap = 256;           // list entries a row keeps between chunks
constexpr int kLinLds = 1024;          // LDS list entries per wavefront while a chunk streams
constexpr int kLinRound = 2;           // 128-bit units per lane per streaming round
constexpr int kLinHeader = 32;         // bytes of a row's state header
constexpr int64_t kLinRowBytes = kLinHeader + 8 * kLinCap;
constexpr int kLinOverflow = 1;        // header flag: the row takes the materialised path

struct LinHead {
  float m;      // running maximum
  float t;      // lower bound of tau: every support entry is > t
  int n;        // list entries
  float zy;     // the label's logit (NaN until its chunk arrives)
  int flags;
  int pad[3];
};

__device__ __forceinline__ LinHead* lin_head(char* state, int64_t r) {
  return reinterpret_cast<LinHead*>(state + r * kLinRowBytes);
}
__device__ __forceinline__ float* lin_vals(char* state, int64_t r) {
  return reinterpret_cast<float*>(state + r * kLinRowBytes + kLinHeader);
}
__device__ __forceinline__ int* lin_cols(char* state, int64_t r) {
  return reinterpret_cast<int*>(state + r * kLinRowBytes + kLinHeader) + kLinCap;
}

__global__ __launch_bounds__(kBlock) void fwl_lin_begin(char* __restrict__ state, int64_t N) {
  const int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (r >= N) return;
  LinHead* h = lin_head(state, r);
  h->m = -INFINITY;
  h->t = -INFINITY;
  h->n = 0;
  h->zy = NAN;
  h->flags = 0;
}

// Stable in-place compaction of one wavefront's LDS list to its entries > t; returns the count.
__device__ __forceinline__ int lin_filter(float* cl, int* ci, int n, float t, int lane) {
  int out = 0;
  for (int p0 = 0; p0 < n; p0 += kWave) {
    const int p = p0 + lane;
    const float v = p < n ? cl[p] : -INFINITY;
    const int c = p < n ? ci[p] : 0;
    const bool keep = v > t;
    const uint64_t b = ballot(keep);
    __builtin_amdgcn_wave_barrier();   // the batch is read before any of it is overwritten
    if (keep) {
      const int at = out + rank_in(b);
      cl[at] = v;
      ci[at] = c;
    }
    out += __popcll(b);
    __builtin_amdgcn_wave_barrier();
  }
  return out;
}

// Appends the values x[0, K) of this lane (columns col[i]) that are > t; entries past the LDS
// capacity are counted but not kept.
template <int K>
__device__ __forceinline__ int lin_append(float* cl, int* ci, int n, const float* x, const int* col, float t,
                                          int lane) {
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const bool c = x[i] > t;
    const uint64_t b = ballot(c);
    if (b != 0) {
      const int at = n + rank_in(b);
      if (c && at < kLinLds) {
        cl[at] = x[i];
        ci[at] = col[i];
      }
      n += __popcll(b);
    }
  }
  return n;
}

// One vocabulary chunk: one wavefront per row streams the row's Vc logits once.
template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void fwl_lin_chunk(const void* __restrict__ zc, int64_t N, int Vc, int64_t ld,
                                                        int64_t v0, const int64_t* __restrict__ tgt,
                                                        char* __restrict__ state) {
  constexpr int U = kUnit<T, VEC>;
  constexpr int K = kLinRound * U;
  __shared__ float s_val[kWavesPerBlock][kLinLds];
  __shared__ int s_col[kWavesPerBlock][kLinLds];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid;
  if (r >= N) return;   // wavefront-uniform; this kernel has no block barrier
  LinHead* hd = lin_head(state, r);
  const int flags = uniform(hd->flags);
  if (flags & kLinOverflow) return;
  float m = hd->m, t = hd->t;
  const int nprev = uniform(hd->n);
  float* cl = s_val[wid];
  int* ci = s_col[wid];
  const rsrc_t row = make_rsrc(static_cast<const char*>(zc) + r * ld * kElemBytes<T>, (uint32_t)(Vc * kElemBytes<T>));
  const int units = (Vc + U - 1) / U;
  int n = 0;
  bool lost = false;
  for (int u0 = 0; u0 < units; u0 += kWave * kLinRound) {
    float x[K];
    int col[K];
#pragma unroll
    for (int q = 0; q < kLinRound; ++q) load_unit<T, VEC>(row, (uint32_t)(u0 + lane + kWave * q), x + U * q);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int e = U * (u0 + lane + kWave * (i / U)) + i % U;
      col[i] = (int)v0 + e;
      if (e >= Vc) x[i] = -INFINITY;   // past the row (loaded as 0)
    }
    float lm = x[0];
#pragma unroll
    for (int i = 1; i < K; ++i) lm = fmaxf(lm, x[i]);
    const float wm = wave_max_f32(lm);
    if (wm > m) {
      m = wm;
      const float tb = bound_below_max(m);
      if (tb > t) t = tb;
    }
    n = lin_append<K>(cl, ci, n, x, col, t, lane);
    if (n > kLinLds) {
      lost = true;
      break;
    }
    __builtin_amdgcn_wave_barrier();
    if (n > kLinLds / 2) n = lin_filter(cl, ci, n, t, lane);
  }
  // the previous chunks' entries that are still above the bound
  if (!lost) {
    const float* pv = lin_vals(state, r);
    const int* pc = lin_cols(state, r);
    for (int p0 = 0; p0 < nprev; p0 += kWave) {
      const int p = p0 + lane;
      float v = p < nprev ? pv[p] : -INFINITY;
      int c = p < nprev ? pc[p] : 0;
      n = lin_append<1>(cl, ci, n, &v, &c, t, lane);
    }
    if (n > kLinLds) lost = true;
  }
  __builtin_amdgcn_wave_barrier();
  if (!lost) n = lin_filter(cl, ci, n, t, lane);
  // too long for the state: tighten the bound with t <- H({z > t}) (each value is <= tau)
  for (int it = 0; !lost && n > kLinCap && it < 32; ++it) {
    double s;
    int c;
    list_sum_count(cl, n, t, lane, s, c);
    const float tn = rd32((s - 1.0) / (double)c);
    if (!(tn > t)) break;
    t = tn;
    n = lin_filter(cl, ci, n, t, lane);
  }
  if (n > kLinCap) lost = true;
  __builtin_amdgcn_wave_barrier();
  if (!lost) {
    float* pv = lin_vals(state, r);
    int* pc = lin_cols(state, r);
    for (int p = lane; p < n; p += kWave) {
      pv[p] = cl[p];
      pc[p] = ci[p];
    }
  }
  const int64_t y = tgt[r];
  const bool here = y >= v0 && y < v0 + Vc;
  const float zy = here ? load_elem<T>(zc, r * ld + (y - v0)) : 0.0f;
  if (lane == 0) {
    hd->m = m;
    hd->t = t;
    hd->n = lost ? 0 : n;
    hd->flags = flags | (lost ? kLinOverflow : 0);
    if (here) hd->zy = zy;
  }
}

// After the last chunk: tau, kappa, H and the loss of every row from its list, and the support's
// columns (in list order).  Flagged rows and rows without a finite maximum get overflow[r] = 1.
__global__ __launch_bounds__(kBlock) void fwl_lin_finish(const char* __restrict__ state, const int64_t* __restrict__ tgt,
                                                         int64_t N, int64_t V, float* __restrict__ H,
                                                         float* __restrict__ loss, int32_t* __restrict__ kappa,
                                                         int32_t* __restrict__ sup, int32_t* __restrict__ overflow) {
  __shared__ float s_val[kWavesPerBlock][kLinCap];
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid;
  if (r >= N) return;
  char* st = const_cast<char*>(state);
  const LinHead* hd = lin_head(st, r);
  const int n = uniform(hd->n);
  const float m = hd->m, t0 = hd->t, zy = hd->zy;
  const bool bad = (uniform(hd->flags) & kLinOverflow) || n == 0 || !isfinite(m);
  if (bad) {
    if (lane == 0) {
      overflow[r] = 1;
      H[r] = NAN;
      loss[r] = NAN;
      kappa[r] = 0;
    }
    return;
  }
  const float* pv = lin_vals(st, r);
  const int* pc = lin_cols(st, r);
  float* cl = s_val[wid];
  for (int p = lane; p < n; p += kWave) cl[p] = pv[p];
  __builtin_amdgcn_wave_barrier();
  double tau;
  int kap;
  uint64_t support;
  resolve_list(cl, n, t0, m, lane, tau, kap, support);
  const float Hf = rd32(tau);
  int out = 0;
  for (int p0 = 0; p0 < n; p0 += kWave) {
    const int p = p0 + lane;
    const bool keep = p < n && cl[p] > Hf;
    const uint64_t b = ballot(keep);
    if (keep) sup[r * kLinCap + out + rank_in(b)] = pc[p];
    out += __popcll(b);
  }
  const int64_t y = tgt[r];
  if (lane == 0) {
    overflow[r] = 0;
    H[r] = Hf;
    loss[r] = (y >= 0 && y < V) ? (float)((1.0 - (double)zy) + tau) : NAN;
    kappa[r] = kap;
  }
}

// The gradient values of row r, as the fused op writes them (scale s = row_scale[r * stride]):
// inv = (float)(s / kappa) on the support, minus (float)s at the label.
struct LinRowGrad {
  float inv, lab;   // value at a support column that is not the label; value at the label
  bool lab_alone;   // the label is outside the support (its own entry)
};

__device__ __forceinline__ LinRowGrad lin_row_grad(const int32_t* sup, int64_t r, int kap, int64_t y, int64_t V,
                                                   double s, int lane) {
  LinRowGrad g;
  g.inv = (float)(s / (double)kap);
  const float sf = (float)s;
  bool in = false;
  if (y >= 0 && y < V) {
    for (int p0 = 0; p0 < kap; p0 += kWave) {
      const int p = p0 + lane;
      in |= ballot(p < kap && sup[r * kLinCap + p] == (int)y) != 0;
    }
    g.lab = in ? g.inv - sf : 0.0f - sf;
    g.lab_alone = !in;
  } else {
    g.lab = 0.0f;
    g.lab_alone = false;
  }
  return g;
}

// dhidden[r] = sum over the row's non-zero gradient columns j of g_rj * weight[j], accumulated in
// fp32 in support order (the label last when it is outside the support).  One wavefront per row;
// flagged rows (kappa 0) are left to the caller.
template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void fwl_lin_dhidden(const void* __restrict__ W, int64_t V, int d,
                                                          const int64_t* __restrict__ tgt,
                                                          const int32_t* __restrict__ kappa,
                                                          const int32_t* __restrict__ sup,
                                                          const float* __restrict__ rscale, int64_t rs_stride,
                                                          int64_t N, void* __restrict__ dh) {
  constexpr int U = kUnit<T, VEC>;
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid;
  if (r >= N) return;
  const int kap = uniform(kappa[r]);
  if (kap <= 0) return;
  const int64_t y = tgt[r];
  const LinRowGrad g = lin_row_grad(sup, r, kap, y, V, (double)rscale[r * rs_stride], lane);
  const uint32_t row_bytes = (uint32_t)(d * kElemBytes<T>);
  const rsrc_t out = make_rsrc(static_cast<char*>(dh) + r * (int64_t)d * kElemBytes<T>, row_bytes);
  const int units = (d + U - 1) / U;
  for (int u = lane; u - lane < units; u += kWave) {
    float acc[U];
#pragma unroll
    for (int e = 0; e < U; ++e) acc[e] = 0.0f;
    for (int p = 0; p < kap; ++p) {
      const int j = uniform(sup[r * kLinCap + p]);
      if (j < 0 || (int64_t)j >= V) continue;   // not a column of weight (never produced by the chunks)
      const float gj = (int64_t)j == y ? g.lab : g.inv;
      float w[U];
      load_unit<T, VEC>(make_rsrc(static_cast<const char*>(W) + (int64_t)j * d * kElemBytes<T>, row_bytes), (uint32_t)u, w);
#pragma unroll
      for (int e = 0; e < U; ++e) acc[e] = fmaf(gj, w[e], acc[e]);
    }
    if (g.lab_alone) {
      float w[U];
      load_unit<T, VEC>(make_rsrc(static_cast<const char*>(W) + y * d * kElemBytes<T>, row_bytes), (uint32_t)u, w);
#pragma unroll
      for (int e = 0; e < U; ++e) acc[e] = fmaf(g.lab, w[e], acc[e]);
    }
    store_unit<T, VEC>(out, (uint32_t)u, acc);
  }
}

// (column, row) entries of the gradient, one per support column and one per label outside the
// support: key = column * 2N + 2 * row (+ 1 for a label entry), value g.  Row r's entries start
// at offsets[r] (exclusive prefix sum of kappa[r] + [label outside the support]).
__global__ __launch_bounds__(kBlock) void fwl_lin_coo(const int64_t* __restrict__ tgt, int64_t N, int64_t V,
                                                      const int32_t* __restrict__ kappa,
                                                      const int32_t* __restrict__ sup,
                                                      const int64_t* __restrict__ offsets,
                                                      const float* __restrict__ rscale, int64_t rs_stride,
                                                      int64_t* __restrict__ keys, float* __restrict__ vals) {
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + wid;
  if (r >= N) return;
  const int kap = uniform(kappa[r]);
  if (kap <= 0) return;
  const int64_t y = tgt[r];
  const LinRowGrad g = lin_row_grad(sup, r, kap, y, V, (double)rscale[r * rs_stride], lane);
  const int64_t o = offsets[r];
  for (int p = lane; p < kap; p += kWave) {
    int64_t j = sup[r * kLinCap + p];
    if (j < 0 || j >= V) j = V;   // not a column of weight: a key that dweight skips
    keys[o + p] = j * 2 * N + 2 * r;
    vals[o + p] = j == y ? g.lab : g.inv;
  }
  if (g.lab_alone && lane == 0) {
    keys[o + kap] = y * 2 * N + 2 * r + 1;
    vals[o + kap] = g.lab;
  }
}

// dweight[j] = sum of g * hidden[row] over column j's entries, in key order (keys sorted): every
// output element is one fma chain over the column's entries in that order.  The grid strides
// over the entries.  The wavefront at a column's first entry finds the column's end (a galloping
// then binary search over the keys) and, for a column of at most kLinShortColumn entries, does
// the whole column.  A longer column (a frequent label, or many rows sharing support entries) is
// split over the hidden dimension instead: the wavefronts at its first nw entries
// (nw = min(units / 64, 64)) each take every nw-th group of 64 units, with the entries' keys and
// values read through the scalar cache eight at a time and their hidden units loaded eight at a
// time.  Keys of column >= V (padding after the entries) are skipped.
constexpr int64_t kLinDweightBlocks = 65536;
constexpr int64_t kLinShortColumn = 32;
constexpr int kLinBatch = 8;

template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void fwl_lin_dweight(const void* __restrict__ hid, int64_t N, int64_t V, int d,
                                                          const int64_t* __restrict__ keys,
                                                          const float* __restrict__ vals, int64_t P,
                                                          void* __restrict__ dW) {
  constexpr int U = kUnit<T, VEC>;
  const int lane = lane_id();
  const int wid = uniform((int)(threadIdx.x >> 6));
  const int64_t twoN = 2 * N;
  const uint32_t row_bytes = (uint32_t)(d * kElemBytes<T>);
  const int units = (d + U - 1) / U;
  const int groups = (units + kWave - 1) / kWave;        // groups of 64 units
  const int nw = groups < kWave ? groups : kWave;         // wavefronts on a long column
  auto col = [&](int64_t p) { return keys[p] / twoN; };
  auto hrow = [&](int64_t p) {   // the entry's row of hidden (keys >= 0: 0 <= n < N)
    const int64_t n = (keys[p] % twoN) / 2;
    return make_rsrc(static_cast<const char*>(hid) + n * d * kElemBytes<T>, row_bytes);
  };
  for (int64_t p = (int64_t)blockIdx.x * kWavesPerBlock + wid; p < P; p += (int64_t)gridDim.x * kWavesPerBlock) {
    const int64_t j = col(p);
    if (j >= V) break;                                       // padding: sorted after every entry
    if (j < 0) continue;                                     // not a column of weight
    // c: entries of the same column directly before p, counted up to nw (lane i looks at p - 1 - i)
    const int64_t q = p - 1 - lane;
    const uint64_t same = ballot(lane < nw && q >= 0 && col(q) == j);
    const int c = (int)__builtin_ctzll(~same);
    if (c >= nw) continue;                                   // deeper into its column: no work
    const int64_t p0 = p - c;
    // the column's end: galloping from p0, then a binary search
    int64_t lo = p0, step = 1;
    while (lo + step < P && col(lo + step) == j) {
      lo += step;
      step *= 2;
    }
    int64_t hi = lo + step < P ? lo + step : P;
    while (hi - lo > 1) {
      const int64_t mid = lo + (hi - lo) / 2;
      if (col(mid) == j) lo = mid;
      else hi = mid;
    }
    const int64_t p1 = hi;
    const rsrc_t out = make_rsrc(static_cast<char*>(dW) + j * d * kElemBytes<T>, row_bytes);
    if (p1 - p0 <= kLinShortColumn) {
      if (c != 0) continue;
      for (int u = lane; u - lane < units; u += kWave) {
        float acc[U];
#pragma unroll
        for (int e = 0; e < U; ++e) acc[e] = 0.0f;
        for (int64_t pp = p0; pp < p1; ++pp) {
          const float gv = vals[pp];
          float h[U];
          load_unit<T, VEC>(hrow(pp), (uint32_t)u, h);
#pragma unroll
          for (int e = 0; e < U; ++e) acc[e] = fmaf(gv, h[e], acc[e]);
        }
        store_unit<T, VEC>(out, (uint32_t)u, acc);
      }
      continue;
    }
    // a long column: unit groups c, c + nw, ... of it (offsets past the row read 0, stores dropped)
    for (int gi = c; gi < groups; gi += nw) {
      const uint32_t u = (uint32_t)(kWave * gi + lane);
      float acc[U];
#pragma unroll
      for (int e = 0; e < U; ++e) acc[e] = 0.0f;
      for (int64_t pb = p0; pb < p1; pb += kLinBatch) {
        float h[kLinBatch][U];
        float gv[kLinBatch];
#pragma unroll
        for (int k = 0; k < kLinBatch; ++k) {
          const bool in = pb + k < p1;
          gv[k] = in ? vals[pb + k] : 0.0f;
          load_unit<T, VEC>(in ? hrow(pb + k) : make_rsrc(hid, 0u), u, h[k]);
        }
#pragma unroll
        for (int k = 0; k < kLinBatch; ++k) {
          if (pb + k >= p1) break;
#pragma unroll
          for (int e = 0; e < U; ++e) acc[e] = fmaf(gv[k], h[k][e], acc[e]);
        }
      }
      store_unit<T, VEC>(out, u, acc);
    }
  }
}

// ---- the linear layer fused with the loss (host side)

template <typename T>
bool lin_vec_ok(const void* a, const void* b, int64_t d) {
  return (d * kElemBytes<T>) % 16 == 0 && aligned(a, 16) && aligned(b, 16);
}

template <typename T>
int lin_chunk(const void* zc, int64_t N, int64_t Vc, int64_t ld, int64_t v0, const int64_t* y, void* state,
              hipStream_t s) {
  if (!aligned(zc, kElemBytes<T>)) return FWL_ERR_ALIGNMENT;
  const int64_t blocks = (N + kWavesPerBlock - 1) / kWavesPerBlock;
  if ((Vc % kUnit<T, true>) == 0 && (ld % kUnit<T, true>) == 0 && aligned(zc, 16))
    hipLaunchKernelGGL((fwl_lin_chunk<T, true>), dim3((unsigned)blocks), dim3(kBlock), 0, s, zc, N, (int)Vc, ld, v0, y,
                       static_cast<char*>(state));
  else
    hipLaunchKernelGGL((fwl_lin_chunk<T, false>), dim3((unsigned)blocks), dim3(kBlock), 0, s, zc, N, (int)Vc, ld, v0,
                       y, static_cast<char*>(state));
  return launch_status();
}

template <typename T>
int lin_dhidden(const void* W, int64_t V, int64_t d, const int64_t* y, const int32_t* kappa, const int32_t* sup,
                const float* rs, int64_t rs_stride, int64_t N, void* dh, hipStream_t s) {
  if (!aligned(W, kElemBytes<T>) || !aligned(dh, kElemBytes<T>)) return FWL_ERR_ALIGNMENT;
  const int64_t blocks = (N + kWavesPerBlock - 1) / kWavesPerBlock;
  if (lin_vec_ok<T>(W, dh, d))
    hipLaunchKernelGGL((fwl_lin_dhidden<T, true>), dim3((unsigned)blocks), dim3(kBlock), 0, s, W, V, (int)d, y, kappa,
                       sup, rs, rs_stride, N, dh);
  else
    hipLaunchKernelGGL((fwl_lin_dhidden<T, false>), dim3((unsigned)blocks), dim3(kBlock), 0, s, W, V, (int)d, y,
                       kappa, sup, rs, rs_stride, N, dh);
  return launch_status();
}

template <typename T>
int lin_dweight(const void* hid, int64_t N, int64_t V, int64_t d, const int64_t* keys, const float* vals, int64_t P,
                void* dW, hipStream_t s) {
  if (!aligned(hid, kElemBytes<T>) || !aligned(dW, kElemBytes<T>)) return FWL_ERR_ALIGNMENT;
  int64_t blocks = (P + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > kLinDweightBlocks) blocks = kLinDweightBlocks;   // the entries are strided over the grid
  if (lin_vec_ok<T>(hid, dW, d))
    hipLaunchKernelGGL((fwl_lin_dweight<T, true>), dim3((unsigned)blocks), dim3(kBlock), 0, s, hid, N, V, (int)d,
                       keys, vals, P, dW);
  else
    hipLaunchKernelGGL((fwl_lin_dweight<T, false>), dim3((unsigned)blocks), dim3(kBlock), 0, s, hid, N, V, (int)d,
                       keys, vals, P, dW);
  return launch_status();
}

// the linear entry points' dimension limits: rows of the state addressed in 64 bits, columns and
// hidden sizes in 32 bits, and grids within 2^31 blocks
constexpr int64_t kLinMaxV = (int64_t)1 << 30;
constexpr int64_t kLinMaxD = (int64_t)1 << 26;
bool lin_bad_rows(int64_t N) { return N < 0 || N > ((int64_t)1 << 31); }

}  // namespace

// ------------------------------------------------------------------------------------------------
// C ABI

extern "C" {

size_t fwl_linear_state_bytes(int64_t N) { return N > 0 ? (size_t)N * (size_t)kLinRowBytes : 0; }

int fwl_linear_support_cap(void) { return kLinCap; }

int fwl_linear_begin(void* state, int64_t N, hipStream_t stream) {
  if (lin_bad_rows(N) || (N > 0 && state == nullptr)) return FWL_ERR_INVALID_ARG;
  if (!aligned(state, 16)) return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  hipLaunchKernelGGL(fwl_lin_begin, dim3((unsigned)((N + kBlock - 1) / kBlock)), dim3(kBlock), 0, stream,
                     static_cast<char*>(state), N);
  return launch_status();
}

int fwl_linear_chunk(int dtype, const void* logits, int64_t N, int64_t Vc, int64_t ld, int64_t v0, int64_t V,
                     const int64_t* targets, void* state, hipStream_t stream) {
  if (lin_bad_rows(N) || Vc < 1 || Vc > kMaxC || ld < Vc || v0 < 0 || V > kLinMaxV || v0 + Vc > V ||
      (N > 0 && (logits == nullptr || targets == nullptr || state == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(targets, 8) || !aligned(state, 16)) return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  switch (dtype) {
    case FWL_FLOAT32: return lin_chunk<float>(logits, N, Vc, ld, v0, targets, state, stream);
    case FWL_BFLOAT16: return lin_chunk<bf16_t>(logits, N, Vc, ld, v0, targets, state, stream);
    case FWL_FLOAT16: return lin_chunk<f16_t>(logits, N, Vc, ld, v0, targets, state, stream);
    default: return FWL_ERR_INVALID_ARG;
  }
}

int fwl_linear_finish(const void* state, const int64_t* targets, int64_t N, int64_t V, float* H, float* losses,
                      int32_t* kappa, int32_t* support, int32_t* overflow, hipStream_t stream) {
  if (lin_bad_rows(N) || V < 1 || V > kLinMaxV ||
      (N > 0 && (state == nullptr || targets == nullptr || H == nullptr || losses == nullptr || kappa == nullptr ||
                 support == nullptr || overflow == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(state, 16) || !aligned(targets, 8) || !aligned(H, 4) || !aligned(losses, 4) || !aligned(kappa, 4) ||
      !aligned(support, 4) || !aligned(overflow, 4))
    return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  hipLaunchKernelGGL(fwl_lin_finish, dim3((unsigned)((N + kWavesPerBlock - 1) / kWavesPerBlock)), dim3(kBlock), 0,
                     stream, static_cast<const char*>(state), targets, N, V, H, losses, kappa, support, overflow);
  return launch_status();
}

int fwl_linear_dhidden(int dtype, const void* weight, int64_t V, int64_t d, const int64_t* targets,
                       const int32_t* kappa, const int32_t* support, const float* row_scale, int64_t rs_stride,
                       int64_t N, void* dhidden, hipStream_t stream) {
  if (lin_bad_rows(N) || V < 1 || V > kLinMaxV || d < 1 || d > kLinMaxD || rs_stride < 0 ||
      (N > 0 && (weight == nullptr || targets == nullptr || kappa == nullptr || support == nullptr ||
                 row_scale == nullptr || dhidden == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(targets, 8) || !aligned(kappa, 4) || !aligned(support, 4) || !aligned(row_scale, 4))
    return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  switch (dtype) {
    case FWL_FLOAT32: return lin_dhidden<float>(weight, V, d, targets, kappa, support, row_scale, rs_stride, N, dhidden, stream);
    case FWL_BFLOAT16: return lin_dhidden<bf16_t>(weight, V, d, targets, kappa, support, row_scale, rs_stride, N, dhidden, stream);
    case FWL_FLOAT16: return lin_dhidden<f16_t>(weight, V, d, targets, kappa, support, row_scale, rs_stride, N, dhidden, stream);
    default: return FWL_ERR_INVALID_ARG;
  }
}

int fwl_linear_coo(const int64_t* targets, int64_t N, int64_t V, const int32_t* kappa, const int32_t* support,
                   const int64_t* offsets, const float* row_scale, int64_t rs_stride, int64_t* keys, float* values,
                   hipStream_t stream) {
  if (lin_bad_rows(N) || V < 1 || V > kLinMaxV || rs_stride < 0 ||
      (N > 0 && (targets == nullptr || kappa == nullptr || support == nullptr || offsets == nullptr ||
                 row_scale == nullptr || keys == nullptr || values == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(targets, 8) || !aligned(offsets, 8) || !aligned(keys, 8) || !aligned(kappa, 4) || !aligned(support, 4) ||
      !aligned(row_scale, 4) || !aligned(values, 4))
    return FWL_ERR_ALIGNMENT;
  if (N == 0) return FWL_OK;
  hipLaunchKernelGGL(fwl_lin_coo, dim3((unsigned)((N + kWavesPerBlock - 1) / kWavesPerBlock)), dim3(kBlock), 0, stream,
                     targets, N, V, kappa, support, offsets, row_scale, rs_stride, keys, values);
  return launch_status();
}

int fwl_linear_dweight(int dtype, const void* hidden, int64_t N, int64_t V, int64_t d, const int64_t* keys,
                       const float* values, int64_t P, void* dweight, hipStream_t stream) {
  if (lin_bad_rows(N) || V < 1 || V > kLinMaxV || d < 1 || d > kLinMaxD || P < 0 || P > ((int64_t)1 << 32) ||
      (P > 0 && (hidden == nullptr || keys == nullptr || values == nullptr || dweight == nullptr)))
    return FWL_ERR_INVALID_ARG;
  if (!aligned(keys, 8) || !aligned(values, 4)) return FWL_ERR_ALIGNMENT;
  if (P == 0) return FWL_OK;
  switch (dtype) {
    case FWL_FLOAT32: return lin_dweight<float>(hidden, N, V, d, keys, values, P, dweight, stream);
    case FWL_BFLOAT16: return lin_dweight<bf16_t>(hidden, N, V, d, keys, values, P, dweight, stream);
    case FWL_FLOAT16: return lin_dweight<f16_t>(hidden, N, V, d, keys, values, P, dweight, stream);
    default: return FWL_ERR_INVALID_ARG;
  }
}

}  // extern "C"
