// Event index construction and event gather / scatter for gfx950.
//
// Index build (bit-exact, ascending t within each row) with no host synchronisation.  For
// B <= 16384 rows: event_count_kernel, then event_fill_prefix_kernel (below), which folds the prefix
// sum into the fill.  Larger B, three launches:
//   1. event_count_kernel : one wave per row; 64 timesteps per ballot, popcount (the mask loads of up to
//                           1024 steps issued together).
//   2. event_scan_kernel  : one workgroup; exclusive prefix sum of the counts over
//                           tiles of 4096 rows with a running carry; also total
//                           and max count (stats[0], stats[1]).
//   3. event_fill_kernel  : one wave per row again; a lane's rank among the set
//                           bits of the ballot (mbcnt) plus the running count gives
//                           the packed slot of its event.
// Gather / scatter are byte moves over 16/4/2/1-byte units chosen from the row
// size and pointer alignment; every unit looks its source up in the int32 tables,
// so non-event rows are copied exactly and padded rows are exact zeros.
#include "internal.h"

namespace hclsm {

constexpr int EV_WAVES = 4;  // rows (waves) per workgroup in count / fill

__global__ void __launch_bounds__(64 * EV_WAVES)
event_count_kernel(const void* __restrict__ mask, int mdt, int64_t B, int64_t T, int rule,
                   int32_t* __restrict__ counts) {
  const int64_t b = (int64_t)blockIdx.x * EV_WAVES + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= B) return;  // whole wave exits together
  int c = 0;
  for (int64_t t0 = 0; t0 < T; t0 += 64 * MASK_BLOCKS) {
    bool ev[MASK_BLOCKS];
    mask_events<MASK_BLOCKS>(mask, mdt, b, T, t0, lane, rule, ev);
#pragma unroll
    for (int u = 0; u < MASK_BLOCKS; ++u) c += __popcll(__ballot(ev[u]));
  }
  if (lane == 0) counts[b] = c;
}

// Row counts of a [B, T] mask alone (composite entry points that build the rest of the index later).
int event_counts(const void* mask, int mdt, int64_t B, int64_t T, int rule, int32_t* counts, hipStream_t st) {
  if (B <= 0) return 0;
  const unsigned g = (unsigned)((B + EV_WAVES - 1) / EV_WAVES);
  hipLaunchKernelGGL(event_count_kernel, dim3(g), dim3(64 * EV_WAVES), 0, st, mask, mdt, B, T, rule, counts);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

constexpr int SCAN_THREADS = 1024;
constexpr int SCAN_PER_THREAD = 4;

__global__ void __launch_bounds__(SCAN_THREADS)
event_scan_kernel(const int32_t* __restrict__ counts, int64_t B, int32_t* __restrict__ offsets,
                  int32_t* __restrict__ stats) {
  __shared__ int32_t wsum[SCAN_THREADS / 64];
  __shared__ int32_t wmax[SCAN_THREADS / 64];
  __shared__ int32_t carry_s, kmax_s;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) { carry_s = 0; kmax_s = 0; }
  __syncthreads();
  constexpr int64_t TILE = (int64_t)SCAN_THREADS * SCAN_PER_THREAD;
  for (int64_t base = 0; base < B; base += TILE) {
    int32_t v[SCAN_PER_THREAD];
    int32_t local = 0, lmax = 0;
#pragma unroll
    for (int i = 0; i < SCAN_PER_THREAD; ++i) {
      const int64_t j = base + (int64_t)tid * SCAN_PER_THREAD + i;
      v[i] = (j < B) ? counts[j] : 0;
      local += v[i];
      lmax = v[i] > lmax ? v[i] : lmax;
    }
    // inclusive wave scan of `local`
    int32_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    int32_t m = lmax;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int32_t o = __shfl_xor(m, off, 64);
      m = o > m ? o : m;
    }
    if (lane == 63) wsum[wid] = incl;
    if (lane == 0) wmax[wid] = m;
    __syncthreads();
    int32_t wprefix = 0, tile_total = 0, tile_max = 0;
    for (int w = 0; w < SCAN_THREADS / 64; ++w) {
      if (w < wid) wprefix += wsum[w];
      tile_total += wsum[w];
      tile_max = wmax[w] > tile_max ? wmax[w] : tile_max;
    }
    const int32_t carry = carry_s;
    int32_t run = carry + wprefix + incl - local;  // exclusive prefix of this thread's first element
#pragma unroll
    for (int i = 0; i < SCAN_PER_THREAD; ++i) {
      const int64_t j = base + (int64_t)tid * SCAN_PER_THREAD + i;
      if (j < B) offsets[j] = run;
      run += v[i];
    }
    __syncthreads();
    if (tid == 0) {
      carry_s = carry + tile_total;
      kmax_s = tile_max > kmax_s ? tile_max : kmax_s;
    }
    __syncthreads();
  }
  if (tid == 0) {
    offsets[B] = carry_s;
    stats[0] = carry_s;
    stats[1] = kmax_s;
  }
}

// One wave writes row b's part of the tables: slot_of[b, t] (rank among the row's events or -1), and for event
// rank r, indices[off + r] = t and rows[off + r] = b.
__device__ __forceinline__ void fill_row(const void* mask, int mdt, int64_t b, int64_t T, int rule, int lane, int32_t off,
                                         int32_t* __restrict__ indices, int32_t* __restrict__ rows,
                                         int32_t* __restrict__ slot_of) {
  int32_t run = 0;
  for (int64_t t0 = 0; t0 < T; t0 += 64 * MASK_BLOCKS) {
    bool ev[MASK_BLOCKS];
    mask_events<MASK_BLOCKS>(mask, mdt, b, T, t0, lane, rule, ev);
#pragma unroll
    for (int u = 0; u < MASK_BLOCKS; ++u) {
      const int64_t t = t0 + 64 * u + lane;
      const uint64_t bal = __ballot(ev[u]);
      const int32_t rank = (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      if (t < T) {
        if (slot_of) slot_of[b * T + t] = ev[u] ? run + rank : -1;
        if (ev[u]) {
          indices[off + run + rank] = (int32_t)t;
          if (rows) rows[off + run + rank] = (int32_t)b;
        }
      }
      run += __popcll(bal);
    }
  }
}

__global__ void __launch_bounds__(64 * EV_WAVES)
event_fill_kernel(const void* __restrict__ mask, int mdt, int64_t B, int64_t T, int rule,
                  const int32_t* __restrict__ offsets, int32_t* __restrict__ indices,
                  int32_t* __restrict__ rows, int32_t* __restrict__ slot_of) {
  const int64_t b = (int64_t)blockIdx.x * EV_WAVES + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= B) return;
  const int32_t off = offsets[b];
  fill_row(mask, mdt, b, T, rule, lane, off, indices, rows, slot_of);
}

// Fill with the prefix sum folded in (B <= PREFIX_MAX_ROWS): each workgroup sums counts[0, b0) of
// the rows before its own (a few KB from L2), so no separate scan launch is needed; the last
// workgroup also writes offsets[B] and the stats {total, max count}.
constexpr int64_t PREFIX_MAX_ROWS = 16384;

__device__ __forceinline__ int32_t block_sum(int32_t v, int32_t* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int32_t t = 0;
  for (int w = 0; w < EV_WAVES; ++w) t += red[w];
  return t;
}

__global__ void __launch_bounds__(64 * EV_WAVES)
event_fill_prefix_kernel(const void* __restrict__ mask, int mdt, int64_t B, int64_t T, int rule,
                         const int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                         int32_t* __restrict__ indices, int32_t* __restrict__ rows,
                         int32_t* __restrict__ slot_of, int32_t* __restrict__ stats) {
  __shared__ int32_t red[EV_WAVES];
  const int64_t b0 = (int64_t)blockIdx.x * EV_WAVES;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  // counts[0, b0): 8 loads per thread in flight per round (a later workgroup reads up to 16384 counts)
  int32_t s = 0;
  for (int64_t i0 = tid; i0 < b0; i0 += 8 * 64 * EV_WAVES) {
    int32_t c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + (int64_t)u * 64 * EV_WAVES;
      c[u] = i < b0 ? counts[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) s += c[u];
  }
  const int32_t prefix = block_sum(s, red);
  const int64_t b = b0 + wid;
  int32_t off = prefix;
  for (int w = 0; w < wid; ++w) off += (b0 + w < B) ? counts[b0 + w] : 0;
  if (b < B) {
    if (lane == 0) offsets[b] = off;
    fill_row(mask, mdt, b, T, rule, lane, off, indices, rows, slot_of);
  }
  if (blockIdx.x == gridDim.x - 1) {   // totals: every row count, summed and maxed by this workgroup
    int32_t t = 0, m = 0;
    for (int64_t i0 = tid; i0 < B; i0 += 8 * 64 * EV_WAVES) {
      int32_t c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t i = i0 + (int64_t)u * 64 * EV_WAVES;
        c[u] = i < B ? counts[i] : 0;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        t += c[u];
        m = c[u] > m ? c[u] : m;
      }
    }
    const int32_t total = block_sum(t, red);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const int32_t v = __shfl_xor(m, o, 64);
      m = v > m ? v : m;
    }
    __syncthreads();
    if (lane == 0) red[wid] = m;
    __syncthreads();
    if (tid == 0) {
      int32_t mx = 0;
      for (int w = 0; w < EV_WAVES; ++w) mx = red[w] > mx ? red[w] : mx;
      offsets[B] = total;
      stats[0] = total;
      stats[1] = mx;
    }
  }
}

// ---------------------------------------------------------------------------
// byte-unit gather / scatter
// ---------------------------------------------------------------------------

template <typename U> struct Zero;
template <> struct Zero<uint4> { static __device__ uint4 v() { return make_uint4(0u, 0u, 0u, 0u); } };
template <> struct Zero<uint32_t> { static __device__ uint32_t v() { return 0u; } };
template <> struct Zero<uint16_t> { static __device__ uint16_t v() { return 0; } };
template <> struct Zero<uint8_t> { static __device__ uint8_t v() { return 0; } };

// dst[b, k] = k < count[b] ? src[b, indices[offsets[b] + k]] : 0       (rows of `upr` units)
template <typename U>
__global__ void __launch_bounds__(256)
gather_padded_kernel(const U* __restrict__ src, U* __restrict__ dst, int64_t upr, int64_t T, int64_t K,
                     int64_t nunits, const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
                     const int32_t* __restrict__ indices) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < nunits; u += stride) {
    const int64_t r = u / upr, w = u - r * upr;
    const int64_t b = r / K, k = r - b * K;
    U val = Zero<U>::v();
    if (k < counts[b]) {
      const int64_t t = indices[offsets[b] + k];
      val = src[(b * T + t) * upr + w];
    }
    dst[u] = val;
  }
}

// dst[e] = src[rows[e], indices[e]] for e < stats[0]
template <typename U>
__global__ void __launch_bounds__(256)
gather_packed_kernel(const U* __restrict__ src, U* __restrict__ dst, int64_t upr, int64_t T, int64_t capacity,
                     const int32_t* __restrict__ rows, const int32_t* __restrict__ indices,
                     const int32_t* __restrict__ stats) {
  const int64_t total = stats[0] < capacity ? stats[0] : capacity;
  const int64_t nunits = total * upr;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < nunits; u += stride) {
    const int64_t e = u / upr, w = u - e * upr;
    dst[u] = src[((int64_t)rows[e] * T + indices[e]) * upr + w];
  }
}

// out[b, t] = (0 <= s=slot_of[b,t] < K) ? upd[b, s] : base[b, t]   (NULL base / upd read as zeros)
template <typename U>
__global__ void __launch_bounds__(256)
scatter_padded_kernel(const U* base, const U* __restrict__ upd, U* out, int64_t upr, int64_t T,
                      int64_t K, int64_t nunits, const int32_t* __restrict__ slot_of) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < nunits; u += stride) {
    const int64_t r = u / upr, w = u - r * upr;
    const int32_t s = slot_of[r];
    U val = Zero<U>::v();
    if (s >= 0 && s < K) {
      if (upd) val = upd[((r / T) * K + s) * upr + w];
    } else if (base) {
      val = base[u];
    }
    out[u] = val;
  }
}

// out[b, t] = s >= 0 ? packed[offsets[b] + s] : base[b, t]
template <typename U>
__global__ void __launch_bounds__(256)
scatter_packed_kernel(const U* base, const U* __restrict__ packed, U* out, int64_t upr, int64_t T,
                      int64_t nunits, const int32_t* __restrict__ offsets, const int32_t* __restrict__ slot_of) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < nunits; u += stride) {
    const int64_t r = u / upr, w = u - r * upr;
    const int32_t s = slot_of[r];
    U val = Zero<U>::v();
    if (s >= 0) {
      if (packed) val = packed[((int64_t)offsets[r / T] + s) * upr + w];
    } else if (base) {
      val = base[u];
    }
    out[u] = val;
  }
}

static unsigned grid_for(int64_t nunits) {
  int64_t g = (nunits + 255) / 256;
  if (g > 256 * 64) g = 256 * 64;
  return (unsigned)(g < 1 ? 1 : g);
}

// Largest unit (16/4/2/1 bytes) dividing row_bytes and every pointer's alignment.
static int unit_bytes(int64_t row_bytes, std::initializer_list<const void*> ptrs) {
  for (int u : {16, 4, 2}) {
    bool ok = (row_bytes % u) == 0;
    for (const void* p : ptrs) ok = ok && ((((uintptr_t)p) % u) == 0);
    if (ok) return u;
  }
  return 1;
}

// Runs F.template operator()<U>() with U the unit type for `ub` bytes.
template <typename F>
static void with_unit(int ub, F&& f) {
  switch (ub) {
    case 16: f.template operator()<uint4>(); break;
    case 4: f.template operator()<uint32_t>(); break;
    case 2: f.template operator()<uint16_t>(); break;
    default: f.template operator()<uint8_t>(); break;
  }
}

}  // namespace hclsm

using namespace hclsm;

extern "C" int hclsm_event_index(const void* mask, int mask_dtype, int64_t B, int64_t T, int rule,
                                 int32_t* counts, int32_t* offsets, int32_t* indices, int32_t* rows,
                                 int32_t* slot_of, int32_t* stats, void* stream) {
  if (B < 0 || T < 0 || B * T > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (mask_dtype < HCLSM_F32 || mask_dtype > HCLSM_U8) return HCLSM_ERR_DTYPE;
  if (rule != HCLSM_EVENT_GT_HALF && rule != HCLSM_EVENT_NONZERO) return HCLSM_ERR_MODE;
  if (!offsets || !stats || (B > 0 && !counts) || (B * T > 0 && (!mask || !indices))) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  if (B > 0) {
    const unsigned g = (unsigned)((B + EV_WAVES - 1) / EV_WAVES);
    hipLaunchKernelGGL(event_count_kernel, dim3(g), dim3(64 * EV_WAVES), 0, st, mask, mask_dtype, B, T, rule, counts);
    HCLSM_LAUNCH_CHECK();
  }
  if (B > 0 && B <= PREFIX_MAX_ROWS) {   // two launches: counts, then fill with the prefix folded in
    const unsigned g = (unsigned)((B + EV_WAVES - 1) / EV_WAVES);
    hipLaunchKernelGGL(event_fill_prefix_kernel, dim3(g), dim3(64 * EV_WAVES), 0, st, mask, mask_dtype, B, T, rule,
                       counts, offsets, indices, rows, slot_of, stats);
    HCLSM_LAUNCH_CHECK();
    return 0;
  }
  hipLaunchKernelGGL(event_scan_kernel, dim3(1), dim3(SCAN_THREADS), 0, st, counts, B, offsets, stats);
  HCLSM_LAUNCH_CHECK();
  if (B > 0 && T > 0) {
    const unsigned g = (unsigned)((B + EV_WAVES - 1) / EV_WAVES);
    hipLaunchKernelGGL(event_fill_kernel, dim3(g), dim3(64 * EV_WAVES), 0, st, mask, mask_dtype, B, T, rule,
                       offsets, indices, rows, slot_of);
    HCLSM_LAUNCH_CHECK();
  }
  return 0;
}

extern "C" int hclsm_event_gather(const void* src, void* dst, int64_t row_bytes, int64_t B, int64_t T, int64_t K,
                                  const int32_t* counts, const int32_t* offsets, const int32_t* indices,
                                  void* stream) {
  if (row_bytes < 0 || B < 0 || T < 0 || K < 0) return HCLSM_ERR_SHAPE;
  const int64_t nbytes = B * K * row_bytes;
  if (nbytes == 0) return 0;
  if (!dst || !counts || !offsets || !src || !indices) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int ub = unit_bytes(row_bytes, {src, dst});
  const int64_t upr = row_bytes / ub, nunits = nbytes / ub;
  with_unit(ub, [&]<typename U>() {
    hipLaunchKernelGGL(gather_padded_kernel<U>, dim3(grid_for(nunits)), dim3(256), 0, st,
                       (const U*)src, (U*)dst, upr, T, K, nunits, counts, offsets, indices);
  });
  HCLSM_LAUNCH_CHECK();
  return 0;
}

extern "C" int hclsm_event_gather_packed(const void* src, void* dst, int64_t row_bytes, int64_t B, int64_t T,
                                         int64_t capacity, const int32_t* rows, const int32_t* indices,
                                         const int32_t* stats, void* stream) {
  if (row_bytes < 0 || B < 0 || T < 0 || capacity < 0) return HCLSM_ERR_SHAPE;
  if (capacity == 0 || row_bytes == 0) return 0;
  if (!src || !dst || !rows || !indices || !stats) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int ub = unit_bytes(row_bytes, {src, dst});
  const int64_t upr = row_bytes / ub;
  with_unit(ub, [&]<typename U>() {
    hipLaunchKernelGGL(gather_packed_kernel<U>, dim3(grid_for(capacity * upr)), dim3(256), 0, st,
                       (const U*)src, (U*)dst, upr, T, capacity, rows, indices, stats);
  });
  HCLSM_LAUNCH_CHECK();
  return 0;
}

extern "C" int hclsm_event_scatter(const void* base, const void* updates, void* out, int64_t row_bytes,
                                   int64_t B, int64_t T, int64_t K, const int32_t* slot_of, void* stream) {
  if (row_bytes < 0 || B < 0 || T < 0 || K < 0) return HCLSM_ERR_SHAPE;
  const int64_t nbytes = B * T * row_bytes;
  if (nbytes == 0) return 0;
  if (!out || !slot_of) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int ub = unit_bytes(row_bytes, {base, updates, out});
  const int64_t upr = row_bytes / ub, nunits = nbytes / ub;
  with_unit(ub, [&]<typename U>() {
    hipLaunchKernelGGL(scatter_padded_kernel<U>, dim3(grid_for(nunits)), dim3(256), 0, st,
                       (const U*)base, (const U*)updates, (U*)out, upr, T, K, nunits, slot_of);
  });
  HCLSM_LAUNCH_CHECK();
  return 0;
}

extern "C" int hclsm_event_scatter_packed(const void* base, const void* packed, void* out, int64_t row_bytes,
                                          int64_t B, int64_t T, const int32_t* offsets, const int32_t* slot_of,
                                          void* stream) {
  if (row_bytes < 0 || B < 0 || T < 0) return HCLSM_ERR_SHAPE;
  const int64_t nbytes = B * T * row_bytes;
  if (nbytes == 0) return 0;
  if (!out || !slot_of || !offsets) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int ub = unit_bytes(row_bytes, {base, packed, out});
  const int64_t upr = row_bytes / ub, nunits = nbytes / ub;
  with_unit(ub, [&]<typename U>() {
    hipLaunchKernelGGL(scatter_packed_kernel<U>, dim3(grid_for(nunits)), dim3(256), 0, st,
                       (const U*)base, (const U*)packed, (U*)out, upr, T, nunits, offsets, slot_of);
  });
  HCLSM_LAUNCH_CHECK();
  return 0;
}
