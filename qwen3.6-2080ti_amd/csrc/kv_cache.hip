// Paged KV cache slot writes (append) and logical-order gathers for gfx950.
//
// Both are pure copies, so results are bit-exact by construction.  One
// workgroup handles one (token, row); its threads move the kv_heads*head_dim
// elements of K and of V in 16-byte units when the layout allows it.
#include "qa_common.h"

namespace qa {

struct CopyParams {
  const char* key_src;
  const char* value_src;
  int64_t s_b, s_h, s_s;  // source element strides
  char* kbase;
  char* vbase;
  const int64_t* row_k;
  const int64_t* row_v;
  const int64_t* row_blocks;
  int64_t num_blocks, sB, sP, sG, sT;  // pool element strides
  const void* tables;
  int64_t table_stride, max_blocks;
  const void* starts;
  int64_t start_scalar;
  const void* counts;
  int64_t tokens;  // new tokens per row (append) / valid tokens (gather)
  int Hkv, D, bs;
  int esize;  // element bytes
  int table_i64, starts_i64, counts_i64;
};

__device__ __forceinline__ int64_t read_index(const void* base, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(base)[i] : reinterpret_cast<const int32_t*>(base)[i];
}

// Base pointers, physical block count and head stride of row b's pool (see
// qa_paged_kv: stride_head == 0 with row pointers means row_blocks[b]*stride_block).
__device__ __forceinline__ void pool_bases(const CopyParams& p, int b, char*& kb, char*& vb, int64_t& nblk, int64_t& sG) {
  if (p.row_k != nullptr) {
    kb = reinterpret_cast<char*>(p.row_k[b]);
    vb = reinterpret_cast<char*>(p.row_v[b]);
    nblk = p.row_blocks != nullptr ? p.row_blocks[b] : p.num_blocks;
    sG = p.sG != 0 ? p.sG : nblk * p.sP;
  } else {
    kb = p.kbase + static_cast<int64_t>(b) * p.sB * p.esize;
    vb = p.vbase + static_cast<int64_t>(b) * p.sB * p.esize;
    nblk = p.num_blocks;
    sG = p.sG;
  }
}

// UNIT = bytes per copy step (16, 4 or 2).
template <int UNIT>
__device__ __forceinline__ void copy_unit(char* dst, const char* src) {
  if constexpr (UNIT == 16) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  } else if constexpr (UNIT == 4) {
    *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
  } else {
    *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
  }
}

template <int UNIT>
__global__ __launch_bounds__(256) void kv_append_kernel(CopyParams p) {
  const int64_t s = blockIdx.x;
  const int b = blockIdx.y;
  const int64_t count = p.counts != nullptr ? read_index(p.counts, p.counts_i64, b) : p.tokens;
  if (s >= count) return;
  const int64_t start = p.starts != nullptr ? read_index(p.starts, p.starts_i64, b) : p.start_scalar;
  const int64_t pos = start + s;
  if (pos < 0) return;
  const int64_t logical = pos / p.bs;
  if (logical >= p.max_blocks) return;
  const int64_t phys = read_index(p.tables, p.table_i64, static_cast<int64_t>(b) * p.table_stride + logical);
  char* kb;
  char* vb;
  int64_t nblk, sG;
  pool_bases(p, b, kb, vb, nblk, sG);
  if (phys < 0 || phys >= nblk) return;
  const int64_t slot = pos % p.bs;
  const int units_per_row = p.D * p.esize / UNIT;
  const int total = p.Hkv * units_per_row;
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int h = idx / units_per_row;
    const int c = idx - h * units_per_row;
    const int64_t src_off = (static_cast<int64_t>(b) * p.s_b + h * p.s_h + s * p.s_s) * p.esize + static_cast<int64_t>(c) * UNIT;
    const int64_t dst_off = (phys * p.sP + h * sG + slot * p.sT) * p.esize + static_cast<int64_t>(c) * UNIT;
    copy_unit<UNIT>(kb + dst_off, p.key_src + src_off);
    copy_unit<UNIT>(vb + dst_off, p.value_src + src_off);
  }
}

// Gather: destination (B, Hkv, tokens, D) contiguous, written through kbase/vbase
// reinterpretation: key_src/value_src here are the *outputs*.
template <int UNIT>
__global__ __launch_bounds__(256) void kv_gather_kernel(CopyParams p, char* key_out, char* value_out) {
  const int64_t t = blockIdx.x;
  const int b = blockIdx.y;
  const int64_t logical = t / p.bs;
  int64_t phys = logical < p.max_blocks ? read_index(p.tables, p.table_i64, static_cast<int64_t>(b) * p.table_stride + logical) : -1;
  char* kb;
  char* vb;
  int64_t nblk, sG;
  pool_bases(p, b, kb, vb, nblk, sG);
  const bool ok = phys >= 0 && phys < nblk;
  const int64_t slot = t % p.bs;
  const int units_per_row = p.D * p.esize / UNIT;
  const int total = p.Hkv * units_per_row;
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int h = idx / units_per_row;
    const int c = idx - h * units_per_row;
    const int64_t dst_off = (((static_cast<int64_t>(b) * p.Hkv + h) * p.tokens + t) * p.D) * p.esize + static_cast<int64_t>(c) * UNIT;
    if (ok) {
      const int64_t src_off = (phys * p.sP + h * sG + slot * p.sT) * p.esize + static_cast<int64_t>(c) * UNIT;
      copy_unit<UNIT>(key_out + dst_off, kb + src_off);
      copy_unit<UNIT>(value_out + dst_off, vb + src_off);
    } else {
      if constexpr (UNIT == 16) {
        *reinterpret_cast<uint4*>(key_out + dst_off) = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(value_out + dst_off) = make_uint4(0, 0, 0, 0);
      } else if constexpr (UNIT == 4) {
        *reinterpret_cast<uint32_t*>(key_out + dst_off) = 0u;
        *reinterpret_cast<uint32_t*>(value_out + dst_off) = 0u;
      } else {
        *reinterpret_cast<uint16_t*>(key_out + dst_off) = 0;
        *reinterpret_cast<uint16_t*>(value_out + dst_off) = 0;
      }
    }
  }
}

static int element_bytes(int32_t dtype) {
  switch (dtype) {
    case QA_F32: return 4;
    case QA_BF16: return 2;
    case QA_F16: return 2;
    default: return 0;
  }
}

static bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Largest copy unit every address of the kernel satisfies.
static int pick_unit(const CopyParams& p, std::initializer_list<int64_t> strides, std::initializer_list<const void*> ptrs) {
  const int64_t row_bytes = static_cast<int64_t>(p.D) * p.esize;
  bool ok16 = row_bytes % 16 == 0;
  for (int64_t s : strides) ok16 = ok16 && (s * p.esize) % 16 == 0;
  for (const void* ptr : ptrs) ok16 = ok16 && (ptr == nullptr || aligned16(ptr));
  if (ok16) return 16;
  bool ok4 = row_bytes % 4 == 0;
  for (int64_t s : strides) ok4 = ok4 && (s * p.esize) % 4 == 0;
  for (const void* ptr : ptrs) ok4 = ok4 && (ptr == nullptr || (reinterpret_cast<uintptr_t>(ptr) & 3u) == 0);
  return ok4 ? 4 : 2;
}

static int fill_pool(CopyParams& p, const qa_paged_kv* kv, int32_t head_dim) {
  QA_REQUIRE(kv != nullptr, "kv descriptor is null");
  QA_REQUIRE(kv->kv_heads > 0, "kv_heads must be positive");
  QA_REQUIRE(head_dim > 0, "head_dim must be positive");
  QA_REQUIRE(kv->row_key_ptrs != nullptr || (kv->key != nullptr && kv->value != nullptr), "key/value pools must be non-null");
  p.esize = element_bytes(kv->dtype);
  QA_REQUIRE(p.esize > 0, "unsupported KV dtype %s", dtype_name(kv->dtype));
  p.kbase = reinterpret_cast<char*>(kv->key);
  p.vbase = reinterpret_cast<char*>(kv->value);
  p.row_k = kv->row_key_ptrs;
  p.row_v = kv->row_value_ptrs;
  p.row_blocks = kv->row_blocks;
  p.num_blocks = kv->num_blocks;
  p.sB = kv->stride_batch;
  p.sP = kv->stride_block;
  p.sG = kv->stride_head;
  p.sT = kv->stride_token;
  p.Hkv = kv->kv_heads;
  p.D = head_dim;
  return 0;
}

}  // namespace qa

extern "C" int qa_paged_kv_append(const void* key_new, const void* value_new, int32_t dtype, int64_t src_stride_b,
                                  int64_t src_stride_h, int64_t src_stride_s, int64_t batch, int32_t kv_heads,
                                  int64_t new_tokens, int32_t head_dim, const qa_paged_kv* kv, const void* block_tables,
                                  int32_t table_dtype, int64_t table_stride, int64_t max_blocks, const void* starts,
                                  int32_t starts_dtype, int64_t start_scalar, const void* counts, int32_t counts_dtype,
                                  int32_t block_size, hipStream_t stream) {
  using namespace qa;
  CopyParams p{};
  if (int rc = fill_pool(p, kv, head_dim)) return rc;
  QA_REQUIRE(kv->dtype == dtype, "new KV dtype %s must match the pool dtype %s", dtype_name(dtype), dtype_name(kv->dtype));
  QA_REQUIRE(kv_heads == kv->kv_heads, "new KV heads (%d) must match the pool (%d)", kv_heads, kv->kv_heads);
  QA_REQUIRE(key_new && value_new, "new key/value pointers must be non-null");
  QA_REQUIRE(block_tables != nullptr && is_index_dtype(table_dtype), "block table must be an int32/int64 device array");
  QA_REQUIRE(starts == nullptr || is_index_dtype(starts_dtype), "start positions must be int32/int64");
  QA_REQUIRE(counts == nullptr || is_index_dtype(counts_dtype), "counts must be int32/int64");
  QA_REQUIRE(batch > 0 && batch <= 65535, "batch must be in [1, 65535]");
  QA_REQUIRE(block_size > 0 && max_blocks > 0, "block_size and max_blocks must be positive");
  if (new_tokens == 0) return 0;
  QA_REQUIRE(new_tokens > 0 && new_tokens <= 0x7fffffff, "new_tokens out of range");
  p.key_src = reinterpret_cast<const char*>(key_new);
  p.value_src = reinterpret_cast<const char*>(value_new);
  p.s_b = src_stride_b;
  p.s_h = src_stride_h;
  p.s_s = src_stride_s;
  p.tables = block_tables;
  p.table_stride = table_stride;
  p.max_blocks = max_blocks;
  p.starts = starts;
  p.start_scalar = start_scalar;
  p.counts = counts;
  p.tokens = new_tokens;
  p.bs = block_size;
  p.table_i64 = table_dtype == QA_I64;
  p.starts_i64 = starts_dtype == QA_I64;
  p.counts_i64 = counts_dtype == QA_I64;
  const int unit = pick_unit(p, {src_stride_b, src_stride_h, src_stride_s, p.sB, p.sP, p.sG, p.sT},
                             {key_new, value_new, kv->key, kv->value});
  dim3 grid(static_cast<unsigned>(new_tokens), static_cast<unsigned>(batch));
  // Per-row pool pointers cannot be checked on the host: fall back to 2-byte units then.
  const int use = (kv->row_key_ptrs != nullptr) ? (p.esize == 4 ? 4 : 2) : unit;
  if (use == 16)
    hipLaunchKernelGGL(kv_append_kernel<16>, grid, dim3(256), 0, stream, p);
  else if (use == 4)
    hipLaunchKernelGGL(kv_append_kernel<4>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(kv_append_kernel<2>, grid, dim3(256), 0, stream, p);
  return check_launch("kv_append_kernel");
}

extern "C" int qa_paged_kv_gather(const qa_paged_kv* kv, int32_t head_dim, int64_t batch, const void* block_tables,
                                  int32_t table_dtype, int64_t table_stride, int64_t max_blocks, int64_t valid,
                                  int32_t block_size, void* key_out, void* value_out, hipStream_t stream) {
  using namespace qa;
  CopyParams p{};
  if (int rc = fill_pool(p, kv, head_dim)) return rc;
  QA_REQUIRE(key_out && value_out, "gather outputs must be non-null");
  QA_REQUIRE(block_tables != nullptr && is_index_dtype(table_dtype), "block table must be an int32/int64 device array");
  QA_REQUIRE(batch > 0 && batch <= 65535, "batch must be in [1, 65535]");
  QA_REQUIRE(block_size > 0 && max_blocks > 0, "block_size and max_blocks must be positive");
  if (valid == 0) return 0;
  QA_REQUIRE(valid > 0 && valid <= 0x7fffffff, "valid out of range");
  p.tables = block_tables;
  p.table_stride = table_stride;
  p.max_blocks = max_blocks;
  p.tokens = valid;
  p.bs = block_size;
  p.table_i64 = table_dtype == QA_I64;
  const int unit = pick_unit(p, {p.sB, p.sP, p.sG, p.sT}, {kv->key, kv->value, key_out, value_out});
  const int use = (kv->row_key_ptrs != nullptr) ? (p.esize == 4 ? 4 : 2) : unit;
  dim3 grid(static_cast<unsigned>(valid), static_cast<unsigned>(batch));
  char* ko = reinterpret_cast<char*>(key_out);
  char* vo = reinterpret_cast<char*>(value_out);
  if (use == 16)
    hipLaunchKernelGGL(kv_gather_kernel<16>, grid, dim3(256), 0, stream, p, ko, vo);
  else if (use == 4)
    hipLaunchKernelGGL(kv_gather_kernel<4>, grid, dim3(256), 0, stream, p, ko, vo);
  else
    hipLaunchKernelGGL(kv_gather_kernel<2>, grid, dim3(256), 0, stream, p, ko, vo);
  return check_launch("kv_gather_kernel");
}

// ---------------------------------------------------------------------------
// Device-side block reservation for a batched step.  The free list is an ascending
// int32 array of block ids with a device cursor state = {head, count}: the free ids are
// free_list[head .. head + count).  Rows take new blocks from the front in row order, which
// is the reference's allocation policy (lowest free id first, src/decode_state.py:72-78)
// applied to one request after the other.  One workgroup: a first pass sums the blocks
// every row needs and checks the tables, a second writes them, scanning rows 1024 at a
// time, so the result is all-or-nothing and no host round trip is needed.
namespace qa {

struct ReserveParams {
  void* tables;
  int64_t table_stride, max_blocks;
  void* lengths;  // in: current length; out: length + count
  void* positions;  // out (may be null): the length before the step
  const void* counts;
  int64_t count_scalar;
  const int32_t* free_list;
  int32_t* free_state;  // {head, count}
  int32_t* status;
  int64_t batch, capacity;
  int bs;
  int table_i64, lengths_i64, positions_i64, counts_i64;
};

constexpr int RESERVE_THREADS = 1024;

__device__ __forceinline__ void write_index(void* base, int is64, int64_t i, int64_t v) {
  if (is64)
    reinterpret_cast<int64_t*>(base)[i] = v;
  else
    reinterpret_cast<int32_t*>(base)[i] = static_cast<int32_t>(v);
}

__device__ __forceinline__ int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

__global__ __launch_bounds__(RESERVE_THREADS) void kv_reserve_kernel(ReserveParams p) {
  __shared__ int64_t s_need[RESERVE_THREADS / 64];
  __shared__ int s_bad[RESERVE_THREADS / 64];
  __shared__ int s_scan[RESERVE_THREADS / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t head = p.free_state[0];
  const int64_t avail = p.free_state[1];
  const int64_t len_max = p.lengths_i64 ? INT64_MAX / 2 : 0x7fffffff;

  // pass 1: blocks needed and table / length checks
  int64_t need = 0;
  int bad = 0;
  for (int64_t b = tid; b < p.batch; b += RESERVE_THREADS) {
    const int64_t len = read_index(p.lengths, p.lengths_i64, b);
    const int64_t n = p.counts != nullptr ? read_index(p.counts, p.counts_i64, b) : p.count_scalar;
    if (len < 0 || n < 0 || len > len_max - n) {
      bad |= 4;
      continue;
    }
    const int64_t have = ceil_div64(len, p.bs);
    const int64_t want = ceil_div64(len + n, p.bs);
    if (want > p.max_blocks) bad |= 2;
    need += want - have;
  }
  for (int off = 32; off > 0; off >>= 1) {
    need += __shfl_xor(need, off, 64);
    bad |= __shfl_xor(bad, off, 64);
  }
  if (lane == 0) {
    s_need[wave] = need;
    s_bad[wave] = bad;
  }
  __syncthreads();
  int64_t total = 0;
  bad = 0;
#pragma unroll
  for (int w = 0; w < RESERVE_THREADS / 64; ++w) {
    total += s_need[w];
    bad |= s_bad[w];
  }
  int code = 0;
  if (head < 0 || avail < 0 || head + avail > p.capacity) code = 3;  // corrupt cursor
  else if (bad & 4) code = 4;                                         // negative length/count or overflow
  else if (bad & 2) code = 2;                                         // a table is too short
  else if (total > avail) code = 1;                                   // not enough free blocks
  if (code != 0) {
    if (tid == 0) p.status[0] = code;
    return;
  }

  // pass 2: exclusive scan of the per-row block counts, 1024 rows at a time
  int64_t base = head;
  for (int64_t r0 = 0; r0 < p.batch; r0 += RESERVE_THREADS) {
    const int64_t b = r0 + tid;
    int64_t len = 0, n = 0, have = 0;
    int k = 0;
    if (b < p.batch) {
      len = read_index(p.lengths, p.lengths_i64, b);
      n = p.counts != nullptr ? read_index(p.counts, p.counts_i64, b) : p.count_scalar;
      have = ceil_div64(len, p.bs);
      k = static_cast<int>(ceil_div64(len + n, p.bs) - have);
    }
    int incl = k;
    for (int off = 1; off < 64; off <<= 1) {
      const int up = __shfl_up(incl, off, 64);
      if (lane >= off) incl += up;
    }
    if (lane == 63) s_scan[wave] = incl;
    __syncthreads();
    int before = 0, tile = 0;
#pragma unroll
    for (int w = 0; w < RESERVE_THREADS / 64; ++w) {
      const int s = s_scan[w];
      before += w < wave ? s : 0;
      tile += s;
    }
    const int64_t first = base + before + incl - k;
    for (int i = 0; i < k; ++i)
      write_index(p.tables, p.table_i64, b * p.table_stride + have + i, p.free_list[first + i]);
    if (b < p.batch) {
      if (p.positions != nullptr) write_index(p.positions, p.positions_i64, b, len);
      write_index(p.lengths, p.lengths_i64, b, len + n);
    }
    base += tile;
    __syncthreads();  // s_scan is reused by the next group of rows
  }
  if (tid == 0) {
    p.free_state[0] = static_cast<int32_t>(head + total);
    p.free_state[1] = static_cast<int32_t>(avail - total);
    p.status[0] = 0;
  }
}

}  // namespace qa

extern "C" int qa_paged_kv_reserve(void* block_tables, int32_t table_dtype, int64_t table_stride, int64_t max_blocks,
                                   void* lengths, int32_t lengths_dtype, void* positions, int32_t positions_dtype,
                                   const void* counts, int32_t counts_dtype, int64_t count_scalar, int64_t batch,
                                   int32_t block_size, const int32_t* free_list, int64_t free_capacity, int32_t* free_state,
                                   int32_t* status, hipStream_t stream) {
  using namespace qa;
  QA_REQUIRE(block_tables != nullptr && is_index_dtype(table_dtype), "block table must be an int32/int64 device array");
  QA_REQUIRE(lengths != nullptr && is_index_dtype(lengths_dtype), "lengths must be an int32/int64 device array");
  QA_REQUIRE(positions == nullptr || is_index_dtype(positions_dtype), "positions must be an int32/int64 device array");
  QA_REQUIRE(counts == nullptr || is_index_dtype(counts_dtype), "counts must be an int32/int64 device array");
  QA_REQUIRE(counts != nullptr || count_scalar >= 0, "count must be non-negative");
  QA_REQUIRE(free_list != nullptr && free_state != nullptr && status != nullptr, "free list, free state and status must be non-null");
  QA_REQUIRE(free_capacity > 0 && free_capacity <= 0x7fffffff, "free list capacity must be in [1, 2^31)");
  QA_REQUIRE(batch >= 0, "batch must be non-negative");
  QA_REQUIRE(block_size > 0 && max_blocks > 0, "block_size and max_blocks must be positive");
  QA_REQUIRE(table_stride >= max_blocks || batch <= 1, "table rows overlap: stride %lld < max_blocks %lld",
             static_cast<long long>(table_stride), static_cast<long long>(max_blocks));
  ReserveParams p{};
  p.tables = block_tables;
  p.table_stride = table_stride;
  p.max_blocks = max_blocks;
  p.lengths = lengths;
  p.positions = positions;
  p.counts = counts;
  p.count_scalar = count_scalar;
  p.free_list = free_list;
  p.free_state = free_state;
  p.status = status;
  p.batch = batch;
  p.capacity = free_capacity;
  p.bs = block_size;
  p.table_i64 = table_dtype == QA_I64;
  p.lengths_i64 = lengths_dtype == QA_I64;
  p.positions_i64 = positions_dtype == QA_I64;
  p.counts_i64 = counts_dtype == QA_I64;
  {
    KernelTimer timer_("kv_reserve", stream);
    hipLaunchKernelGGL(kv_reserve_kernel, dim3(1), dim3(RESERVE_THREADS), 0, stream, p);
  }
  return check_launch("paged_kv_reserve");
}
