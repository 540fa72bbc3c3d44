// topk.hip -- the top-n tokens of logits rows with their softmax probabilities.
//
// For each row r of n logits: scaled = logits * (1 / temperature) when
// temperature > 0 and != 1 (else the logits as they are); p = softmax(scaled),
// computed as exp(scaled - max) * (1 / sum); ids[r, j], probs[r, j] for
// j < min(top_n, n) are the top_n tokens by probability, largest first, ties
// to the lower index.  A row whose maximum is not finite, whose sum is not
// finite or not positive, or that holds a NaN gives the uniform distribution
// 1 / n, i.e. ids 0, 1, 2, ... .  This is Sampler::get_top_tokens
// (src/runtime/sampler.cpp:141-197; the same softmax as Sampler::sample,
// :31-63) on the device: the reference's generator copies the whole logits
// row to the host per token instead (examples/generate_cuda.cpp:81-94).  Where
// the reference leaves the order of equal probabilities to std::partial_sort,
// the order here is the logit, then the index.
//
// Two launches.  Pass 1 (grid chunks x rows, 256 threads): a workgroup reads a
// 2048-value chunk once, forms 64-bit keys (order(value) << 32 | ~index: the
// largest key is the largest value with the smallest index) and keeps its
// top_n keys, plus the chunk's maximum, its sum of exp(value - maximum) and a
// NaN flag.  Pass 2 (one 1024-thread workgroup per row): merges the chunk
// statistics in a fixed order (max, then the sum of sum_c * exp(max_c - max)),
// selects the top_n of the chunks' candidate keys and writes ids and
// probabilities.
//
// Selection (both passes): a radix select over the keys' upper 32 bits (four
// 8-bit digit histograms in LDS, most significant first) finds the top_n-th
// largest value T; the keys >= T (T's ties included) are gathered and sorted by
// one wave in registers (bitonic network, lane shuffles, no barriers), and the
// first top_n are the result.  If more than 256 keys reach T (massive ties) the
// whole set is sorted in LDS instead.  Results are deterministic: the keys are
// distinct, so the sorted order does not depend on the order of gathering.
#include "../launch.hpp"

namespace mle {
namespace {

constexpr int kChunk = 2048;           // values per pass-1 workgroup
constexpr int kP1Threads = 256;
constexpr int kP2Threads = 1024;
constexpr int kP2Keys = 16384;         // candidate keys a row can merge (128 KB of LDS)

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t i) {
  if (v != v) return 0;      // NaN (the row becomes uniform anyway)
  if (v == 0.0f) v = 0.0f;   // -0 -> +0
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)~i;
}

__device__ __forceinline__ float key_value(uint64_t k) {
  uint32_t u = (uint32_t)(k >> 32);
  u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
  return __builtin_bit_cast(float, u);
}

// In-place descending bitonic sort of nk (a power of two) keys by NT threads.
template <int NT>
__device__ void bitonic_desc(uint64_t* s, int nk) {
  for (int size = 2; size <= nk; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < nk / 2; i += NT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = s[lo], b = s[hi];
        if ((a < b) == desc) {
          s[lo] = b;
          s[hi] = a;
        }
      }
      __syncthreads();
    }
}

template <int NT, typename T, typename Op>
__device__ T block_reduce(T v, Op op, T* part) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = op(v, __shfl_xor(v, off, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // part[] may still be read from an earlier reduction
  if (lane == 0) part[wave] = v;
  __syncthreads();
  T r = part[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) r = op(r, part[i]);
  return r;
}

struct SelectLds {
  uint32_t hist[256];
  uint64_t cand[256];
  uint32_t digit, above, eq, total, ncand;
};

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Descending bitonic sort of 256 keys held by one wave, 4 per lane (element
// 4 lane + j), in registers.
__device__ void wave_sort256_desc(uint64_t (&v)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 256; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int e = 4 * lane + j;
          const uint64_t o = shfl_xor64(v[j], stride >> 2);
          const bool lower = (e & stride) == 0;
          const bool keep_max = lower == ((e & size) == 0);
          v[j] = keep_max ? (o > v[j] ? o : v[j]) : (o < v[j] ? o : v[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (j & stride) continue;  // handle each in-lane pair once, from its lower element
          const int e = 4 * lane + j;
          const bool desc = (e & size) == 0;
          const uint64_t a = v[j], c = v[j + stride];
          const bool swap = desc ? a < c : a > c;
          v[j] = swap ? c : a;
          v[j + stride] = swap ? a : c;
        }
      }
    }
}

// Top k (k <= kTopTokensMax) of the keys held E per thread by NT threads
// (0 = no key), written sorted descending to out[0, k) (zeros past the number
// of keys).  `full` (NT * E keys of LDS) is used only when more than 256 keys
// tie at the threshold.
template <int NT, int E>
__device__ void select_top(const uint64_t (&key)[E], int k, uint64_t* __restrict__ out,
                           SelectLds& sm, uint64_t* full) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t prefix = 0, mask = 0;
  int need = k;
  bool all = false;  // fewer keys than k: every key is a candidate
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += NT) sm.hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t u = (uint32_t)(key[e] >> 32);
      if (key[e] != 0 && (u & mask) == prefix) atomicAdd(&sm.hist[(u >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      uint32_t h[4], local = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        h[t] = sm.hist[255 - (4 * lane + t)];
        local += h[t];
      }
      uint32_t incl = local;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
        if (lane >= off) incl += o;
      }
      uint32_t run = incl - local;  // keys in the bins above this lane's first bin
      if (lane == 63) sm.total = incl;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (run < (uint32_t)need && (uint32_t)need <= run + h[t]) {
          sm.digit = 255u - (uint32_t)(4 * lane + t);
          sm.above = run;
          sm.eq = h[t];
        }
        run += h[t];
      }
    }
    __syncthreads();
    if (shift == 24 && sm.total <= (uint32_t)k) {
      all = true;
      break;
    }
    need -= (int)sm.above;
    prefix |= sm.digit << shift;
    mask |= 255u << shift;
  }
  // Candidates: every key (all) or the keys with value >= T = prefix.
  const uint32_t ncand = all ? sm.total : (uint32_t)(k - need) + sm.eq;
  if (ncand <= 256) {
    if (tid == 0) sm.ncand = 0;
    for (int i = tid; i < 256; i += NT) sm.cand[i] = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t u = (uint32_t)(key[e] >> 32);
      if (key[e] != 0 && (all || u >= prefix)) sm.cand[atomicAdd(&sm.ncand, 1u)] = key[e];
    }
    __syncthreads();
    if (wave == 0) {
      uint64_t v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = sm.cand[4 * lane + j];
      wave_sort256_desc(v);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * lane + j < k) out[4 * lane + j] = v[j];
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) full[tid * E + e] = key[e];
    __syncthreads();
    bitonic_desc<NT>(full, NT * E);
    for (int j = tid; j < k; j += NT) out[j] = full[j];
  }
  __syncthreads();
}

// Pass 1: workgroup (c, r) over logits[r, c * kChunk : (c + 1) * kChunk).
// keys: [row][chunk][k]; stats: [row][chunk] x {max, sum, nan, 0}.
__global__ __launch_bounds__(kP1Threads) void topk_chunks_kernel(
    const float* __restrict__ x, int64_t n, int k, float inv_temp, int scale,
    uint64_t* __restrict__ keys, float* __restrict__ stats) {
  __shared__ uint64_t s[kChunk];  // only for massive ties
  __shared__ SelectLds sm;
  __shared__ uint64_t top[kTopTokensMax];
  __shared__ float fpart[kP1Threads / 64];
  __shared__ int ipart[kP1Threads / 64];
  const int64_t r = blockIdx.y;
  const int64_t b = (int64_t)blockIdx.x * kChunk;
  const float* row = x + r * n;
  constexpr int PER = kChunk / kP1Threads;
  float v[PER];
  uint64_t key[PER];
  float mx = -__builtin_inff();
  int nan = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t i = b + threadIdx.x + kP1Threads * j;
    float t = -__builtin_inff();
    key[j] = 0;
    if (i < n) {
      t = row[i];
      if (scale) t *= inv_temp;
      key[j] = topk_key(t, (uint32_t)i);
      nan |= t != t;
      mx = fmaxf(mx, t);  // ignores NaN
    }
    v[j] = t;
  }
  mx = block_reduce<kP1Threads>(mx, [](float a, float c) { return fmaxf(a, c); }, fpart);
  nan = block_reduce<kP1Threads>(nan, [](int a, int c) { return a | c; }, ipart);
  float sum = 0.0f;
  if (mx > -__builtin_inff() && mx < __builtin_inff()) {
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (v[j] == v[j]) sum += expf(v[j] - mx);
  }
  sum = block_reduce<kP1Threads>(sum, [](float a, float c) { return a + c; }, fpart);
  select_top<kP1Threads, PER>(key, k, top, sm, s);
  const int64_t slot = r * gridDim.x + blockIdx.x;
  for (int j = threadIdx.x; j < k; j += kP1Threads) keys[slot * k + j] = top[j];
  if (threadIdx.x == 0) {
    stats[slot * 4 + 0] = mx;
    stats[slot * 4 + 1] = sum;
    stats[slot * 4 + 2] = nan ? 1.0f : 0.0f;
    stats[slot * 4 + 3] = 0.0f;
  }
}

// Pass 2: one workgroup per row over its chunks' statistics and candidates.
__global__ __launch_bounds__(kP2Threads) void topk_final_kernel(
    const uint64_t* __restrict__ keys, const float* __restrict__ stats, int chunks, int k,
    int64_t n, int kk, int32_t* __restrict__ ids, float* __restrict__ probs) {
  __shared__ uint64_t s[kP2Keys];  // only for massive ties
  __shared__ SelectLds sm;
  __shared__ uint64_t top[kTopTokensMax];
  __shared__ float fpart[kP2Threads / 64];
  __shared__ int ipart[kP2Threads / 64];
  const int64_t r = blockIdx.x;
  const float* st = stats + r * chunks * 4;
  float mx = -__builtin_inff();
  int bad = 0;
  for (int c = threadIdx.x; c < chunks; c += kP2Threads) {
    mx = fmaxf(mx, st[c * 4 + 0]);
    bad |= st[c * 4 + 2] != 0.0f;
  }
  mx = block_reduce<kP2Threads>(mx, [](float a, float c) { return fmaxf(a, c); }, fpart);
  bad = block_reduce<kP2Threads>(bad, [](int a, int c) { return a | c; }, ipart);
  float sum = 0.0f;
  const bool finite_max = mx > -__builtin_inff() && mx < __builtin_inff();
  if (finite_max) {
    for (int c = threadIdx.x; c < chunks; c += kP2Threads) {
      const float mc = st[c * 4 + 0];
      if (mc > -__builtin_inff()) sum += st[c * 4 + 1] * expf(mc - mx);
    }
  }
  sum = block_reduce<kP2Threads>(sum, [](float a, float c) { return a + c; }, fpart);
  const bool uniform = bad || !finite_max || !(sum > 0.0f) || !(sum < __builtin_inff());
  int32_t* oid = ids + r * kk;
  float* opr = probs + r * kk;
  if (uniform) {
    const float u = 1.0f / (float)n;
    for (int j = threadIdx.x; j < kk; j += kP2Threads) {
      oid[j] = j;
      opr[j] = u;
    }
    return;
  }
  const int total = chunks * k;
  const uint64_t* kr = keys + r * (int64_t)total;
  constexpr int PER = kP2Keys / kP2Threads;
  uint64_t key[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int j = threadIdx.x + kP2Threads * e;
    key[e] = j < total ? kr[j] : 0;
  }
  select_top<kP2Threads, PER>(key, kk, top, sm, s);
  const float inv_sum = 1.0f / sum;
  for (int j = threadIdx.x; j < kk; j += kP2Threads) {
    const uint64_t kv = top[j];
    oid[j] = (int32_t)~(uint32_t)kv;
    opr[j] = expf(key_value(kv) - mx) * inv_sum;
  }
}

}  // namespace

int topk_chunks(int64_t n) { return (int)((n + kChunk - 1) / kChunk); }

int topk_max_n(int k) {
  // Candidate keys of a row must fit pass 2's LDS: chunks * k <= kP2Keys.
  return k <= 0 ? 0 : (kP2Keys / k) * kChunk;
}

hipError_t launch_top_tokens(const float* x, int rows, int64_t n, int top_n, float temperature,
                             int32_t* ids, float* probs, float* workspace, hipStream_t stream) {
  const int kk = (int)(top_n < n ? top_n : n);
  if (rows <= 0 || rows > 65535 || n <= 0 || top_n <= 0 || top_n > kTopTokensMax ||
      n > topk_max_n(kk))
    return hipErrorInvalidValue;
  const int chunks = topk_chunks(n);
  uint64_t* keys = reinterpret_cast<uint64_t*>(workspace);
  float* stats = workspace + (size_t)rows * chunks * kk * 2;
  const bool scale = temperature > 0.0f && temperature != 1.0f;
  const float inv_temp = scale ? 1.0f / temperature : 1.0f;
  hipLaunchKernelGGL(topk_chunks_kernel, dim3((unsigned)chunks, (unsigned)rows), dim3(kP1Threads),
                     0, stream, x, n, kk, inv_temp, scale ? 1 : 0, keys, stats);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(topk_final_kernel, dim3((unsigned)rows), dim3(kP2Threads), 0, stream, keys,
                     stats, chunks, kk, n, kk, ids, probs);
  return hipGetLastError();
}

size_t top_tokens_workspace_floats(int rows, int64_t n, int top_n) {
  const int kk = (int)(top_n < n ? top_n : n);
  const size_t chunks = (size_t)topk_chunks(n);
  return (size_t)rows * chunks * ((size_t)kk * 2 + 4);
}

}  // namespace mle
