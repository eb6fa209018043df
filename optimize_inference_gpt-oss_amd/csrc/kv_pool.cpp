// Paged KV pool: device storage of every layer's cache plus the host
// bookkeeping of blocks and sequences.
//
// Replaces the reference engine's per-layer contiguous caches
// (GpuLayer::kc16/vq8/vs, getp-csrc/engine/gpu_engine.hpp:59-78, allocated in
// gpu_alloc_state :316-334 with slots = max_pos or the window, rounded to 64)
// by 16-token blocks handed out from a free list:
//   full layers    one block id covers 16 positions of a sequence in every full
//                  layer; per layer K and V [num_blocks][Hkv][1024] bf16 in
//                  the block layouts of kv_append.hpp (32 KB per block at Hkv=8)
//   window layers  a ring of W/16 blocks per sequence id, fixed at create time
//                  (the reference's slots = window, gpu_engine.hpp:318-319)
//   tables         int32 [max_seqs][ceil(max_seq_len/16)] and [max_seqs][W/16],
//                  mirrored on the host; gkv_pool_sync uploads the entries that
//                  changed since the last sync, without waiting
// Sizing: num_blocks explicit, or derived from a byte budget, by default 90%
// of the free device memory (288 GB HBM3E on MI355X), instead of the
// reference's halve-the-batch-until-it-fits loop (gpu_fit_batch :425-433).
// Errors are returned, never exit()ed (the reference's HIP_CHECK exits,
// :41-49).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <new>
#include <numeric>
#include <random>
#include <vector>

#include "gkv.h"

namespace {
constexpr int kBT = 16;
constexpr int kD = 64;
} // namespace

struct gkv_pool {
  gkv_pool_config cfg{};
  std::vector<int> layer_index; // layer -> index among full or window layers
  std::vector<char> layer_is_window;
  int n_full = 0, n_window = 0;
  int table_stride = 0; // full-table entries per sequence
  int ring_blocks = 0;  // W / 16
  int64_t num_blocks = 0, num_ring_blocks = 0;
  std::vector<void *> k_full, v_full, k_ring, v_ring;
  std::vector<void *> s_full, s_ring; // fp32 V scales (int8 V only)
  int32_t *d_table = nullptr, *d_ring_table = nullptr;
  std::vector<int32_t> h_table, h_ring_table;
  std::vector<int32_t> free_blocks; // stack; back() is handed out next
  std::vector<int32_t> seq_blocks;  // blocks held per sequence
  std::vector<char> seq_live;
  std::vector<int32_t> free_seqs;
  int64_t device_bytes = 0;
  // Incremental sync: the full-table entries changed since the last sync,
  // as (index, value); they go to the device through one of two pinned
  // staging buffers (reused only once the copy out of it has completed) and
  // a scatter kernel. The first sync uploads the whole tables.
  std::vector<int2> pending;
  bool whole = true;
  int2 *h_stage[2] = {nullptr, nullptr};
  int2 *d_stage[2] = {nullptr, nullptr};
  hipEvent_t stage_done[2] = {nullptr, nullptr};
  size_t stage_cap = 0; // entries per staging buffer
  int stage_i = 0;

  void free_stage() {
    for (int i = 0; i < 2; i++) {
      if (stage_done[i]) {
        (void)hipEventSynchronize(stage_done[i]);
        (void)hipEventDestroy(stage_done[i]);
      }
      if (h_stage[i])
        (void)hipHostFree(h_stage[i]);
      if (d_stage[i])
        (void)hipFree(d_stage[i]);
      h_stage[i] = nullptr;
      d_stage[i] = nullptr;
      stage_done[i] = nullptr;
    }
    stage_cap = 0;
  }

  ~gkv_pool() {
    free_stage();
    for (auto *vec : {&k_full, &v_full, &k_ring, &v_ring, &s_full, &s_ring})
      for (void *p : *vec)
        if (p)
          (void)hipFree(p);
    if (d_table)
      (void)hipFree(d_table);
    if (d_ring_table)
      (void)hipFree(d_ring_table);
  }
};

// Bytes of one 16-token block of one layer: K bf16 (or e4m3), V bf16 (or int8
// or e4m3 codes) + fp32 scales (V's, or K's and V's).
static int64_t k_bytes(int n_kv_heads, int v_format) {
  return (int64_t)n_kv_heads * kBT * kD * (v_format == GKV_KV_FP8 ? 1 : 2);
}
static int64_t v_bytes(int n_kv_heads, int v_format) {
  return (int64_t)n_kv_heads * kBT * kD * (v_format == GKV_V_BF16 ? 2 : 1);
}
static int64_t s_bytes(int n_kv_heads, int v_format) {
  return (int64_t)n_kv_heads * kBT * 4 *
         (v_format == GKV_V_INT8 ? 1 : v_format == GKV_KV_FP8 ? 2 : 0);
}
static int64_t block_bytes_per_layer(int n_kv_heads, int v_format) {
  return k_bytes(n_kv_heads, v_format) + v_bytes(n_kv_heads, v_format) +
         s_bytes(n_kv_heads, v_format);
}

extern "C" int gkv_pool_create(const gkv_pool_config *cfg, gkv_pool **out) {
  if (!cfg || !out)
    return GKV_ERR_ARG;
  *out = nullptr;
  const gkv_pool_config &c = *cfg;
  if (c.n_layers <= 0 || c.n_kv_heads <= 0 || c.max_seqs <= 0 || c.max_seq_len <= 0 ||
      c.window < 0 || c.num_blocks < 0 || c.bytes_budget < 0)
    return GKV_ERR_ARG;
  if (c.head_dim != kD || c.window % kBT != 0)
    return GKV_ERR_UNSUPPORTED;
  if (c.v_format != GKV_V_BF16 && c.v_format != GKV_V_INT8 && c.v_format != GKV_KV_FP8)
    return GKV_ERR_ARG;
  gkv_pool *p = new (std::nothrow) gkv_pool();
  if (!p)
    return GKV_ERR_CAPACITY;
  p->cfg = c;
  p->layer_index.resize(c.n_layers);
  p->layer_is_window.resize(c.n_layers);
  for (int l = 0; l < c.n_layers; l++) {
    const bool win = c.window > 0 && l % 2 == 0; // run.cpp:617 (l % 2 == 0)
    p->layer_is_window[l] = win;
    p->layer_index[l] = win ? p->n_window++ : p->n_full++;
  }
  p->table_stride = (c.max_seq_len + kBT - 1) / kBT;
  p->ring_blocks = c.window / kBT;
  p->num_ring_blocks = (int64_t)c.max_seqs * p->ring_blocks;
  const int64_t bpl = block_bytes_per_layer(c.n_kv_heads, c.v_format);
  const int64_t ring_bytes = p->num_ring_blocks * bpl * p->n_window;
  const int64_t table_bytes =
      ((int64_t)c.max_seqs * p->table_stride + (int64_t)c.max_seqs * p->ring_blocks) * 4;

  int64_t nb = c.num_blocks;
  if (nb == 0 && p->n_full > 0) {
    int64_t budget = c.bytes_budget;
    if (budget == 0) {
      size_t free_b = 0, total_b = 0;
      if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        delete p;
        return GKV_ERR_HIP;
      }
      budget = (int64_t)(0.9 * (double)free_b);
    }
    nb = (budget - ring_bytes - table_bytes) / (bpl * p->n_full);
    if (nb <= 0) {
      delete p;
      return GKV_ERR_CAPACITY;
    }
  }
  if (nb > INT32_MAX || p->num_ring_blocks > INT32_MAX) {
    delete p;
    return GKV_ERR_CAPACITY;
  }
  p->num_blocks = p->n_full > 0 ? nb : 0;

  auto dev_alloc = [&](void **ptr, int64_t bytes) -> bool {
    if (bytes == 0) {
      *ptr = nullptr;
      return true;
    }
    if (hipMalloc(ptr, (size_t)bytes) != hipSuccess) {
      *ptr = nullptr;
      (void)hipGetLastError();
      return false;
    }
    p->device_bytes += bytes;
    return true;
  };
  const int64_t kb = k_bytes(c.n_kv_heads, c.v_format), vb = v_bytes(c.n_kv_heads, c.v_format);
  const int64_t sb = s_bytes(c.n_kv_heads, c.v_format);
  bool ok = true;
  p->k_full.assign(p->n_full, nullptr);
  p->v_full.assign(p->n_full, nullptr);
  p->s_full.assign(p->n_full, nullptr);
  p->k_ring.assign(p->n_window, nullptr);
  p->v_ring.assign(p->n_window, nullptr);
  p->s_ring.assign(p->n_window, nullptr);
  for (int i = 0; ok && i < p->n_full; i++)
    ok = dev_alloc(&p->k_full[i], p->num_blocks * kb) &&
         dev_alloc(&p->v_full[i], p->num_blocks * vb) &&
         dev_alloc(&p->s_full[i], p->num_blocks * sb);
  for (int i = 0; ok && i < p->n_window; i++)
    ok = dev_alloc(&p->k_ring[i], p->num_ring_blocks * kb) &&
         dev_alloc(&p->v_ring[i], p->num_ring_blocks * vb) &&
         dev_alloc(&p->s_ring[i], p->num_ring_blocks * sb);
  ok = ok && dev_alloc((void **)&p->d_table, (int64_t)c.max_seqs * p->table_stride * 4);
  if (ok && p->ring_blocks > 0)
    ok = dev_alloc((void **)&p->d_ring_table, (int64_t)c.max_seqs * p->ring_blocks * 4);
  if (!ok) {
    delete p;
    return GKV_ERR_CAPACITY;
  }

  // Unassigned table entries are -1: a kernel that meets one flags it.
  p->h_table.assign((size_t)c.max_seqs * p->table_stride, -1);
  p->h_ring_table.resize((size_t)c.max_seqs * p->ring_blocks);
  std::vector<int32_t> ring_ids(p->num_ring_blocks);
  std::iota(ring_ids.begin(), ring_ids.end(), 0);
  p->free_blocks.resize(p->num_blocks);
  // Stack order: block 0 is handed out first unless shuffled.
  for (int64_t i = 0; i < p->num_blocks; i++)
    p->free_blocks[i] = (int32_t)(p->num_blocks - 1 - i);
  if (c.shuffle_seed != 0) {
    std::mt19937_64 rng(c.shuffle_seed);
    std::shuffle(p->free_blocks.begin(), p->free_blocks.end(), rng);
    std::shuffle(ring_ids.begin(), ring_ids.end(), rng);
  }
  std::copy(ring_ids.begin(), ring_ids.end(), p->h_ring_table.begin());
  p->seq_blocks.assign(c.max_seqs, 0);
  p->seq_live.assign(c.max_seqs, 0);
  p->free_seqs.resize(c.max_seqs);
  for (int s = 0; s < c.max_seqs; s++)
    p->free_seqs[s] = c.max_seqs - 1 - s;
  if (gkv_pool_sync(p, nullptr) != GKV_OK || hipDeviceSynchronize() != hipSuccess) {
    delete p;
    return GKV_ERR_HIP;
  }
  *out = p;
  return GKV_OK;
}

extern "C" int gkv_pool_destroy(gkv_pool *pool) {
  if (!pool)
    return GKV_ERR_ARG;
  (void)hipDeviceSynchronize();
  delete pool;
  return GKV_OK;
}

extern "C" int gkv_pool_seq_alloc(gkv_pool *pool, int32_t *seq_id) {
  if (!pool || !seq_id)
    return GKV_ERR_ARG;
  if (pool->free_seqs.empty())
    return GKV_ERR_CAPACITY;
  const int32_t s = pool->free_seqs.back();
  pool->free_seqs.pop_back();
  pool->seq_live[s] = 1;
  pool->seq_blocks[s] = 0;
  *seq_id = s;
  return GKV_OK;
}

extern "C" int gkv_pool_seq_reserve(gkv_pool *pool, int32_t seq_id, int32_t seq_len) {
  if (!pool || seq_len < 0)
    return GKV_ERR_ARG;
  if (seq_id < 0 || seq_id >= pool->cfg.max_seqs || !pool->seq_live[seq_id])
    return GKV_ERR_BLOCK;
  if (pool->n_full == 0)
    return seq_len <= pool->cfg.max_seq_len ? GKV_OK : GKV_ERR_CAPACITY;
  const int32_t need = (seq_len + kBT - 1) / kBT;
  if (need > pool->table_stride)
    return GKV_ERR_CAPACITY;
  const int32_t have = pool->seq_blocks[seq_id];
  if (need <= have)
    return GKV_OK;
  if ((int64_t)(need - have) > (int64_t)pool->free_blocks.size())
    return GKV_ERR_CAPACITY; // nothing taken: all or none
  const size_t base = (size_t)seq_id * pool->table_stride;
  int32_t *row = &pool->h_table[base];
  for (int32_t j = have; j < need; j++) {
    row[j] = pool->free_blocks.back();
    pool->free_blocks.pop_back();
    pool->pending.push_back(int2{(int)(base + j), row[j]});
  }
  pool->seq_blocks[seq_id] = need;
  return GKV_OK;
}

extern "C" int gkv_pool_seq_free(gkv_pool *pool, int32_t seq_id) {
  if (!pool)
    return GKV_ERR_ARG;
  if (seq_id < 0 || seq_id >= pool->cfg.max_seqs || !pool->seq_live[seq_id])
    return GKV_ERR_BLOCK;
  const size_t base = (size_t)seq_id * pool->table_stride;
  int32_t *row = &pool->h_table[base];
  for (int32_t j = pool->seq_blocks[seq_id] - 1; j >= 0; j--) {
    pool->free_blocks.push_back(row[j]);
    row[j] = -1;
    pool->pending.push_back(int2{(int)(base + j), -1});
  }
  pool->seq_blocks[seq_id] = 0;
  pool->seq_live[seq_id] = 0;
  pool->free_seqs.push_back(seq_id);
  return GKV_OK;
}

// Applies n staged (index, value) pairs to the device table, in order (a
// later pair for the same entry wins: each thread takes a distinct pair, and
// the pairs of one entry never repeat within a sync, see gkv_pool_sync).
__global__ void pool_scatter_kernel(int32_t *table, const int2 *pairs, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n)
    table[pairs[i].x] = pairs[i].y;
}

extern "C" int gkv_pool_sync(gkv_pool *pool, void *stream) {
  if (!pool)
    return GKV_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (pool->whole) {
    // the first sync: both tables whole, waited for (create time)
    if (hipMemcpyAsync(pool->d_table, pool->h_table.data(), pool->h_table.size() * 4,
                       hipMemcpyHostToDevice, s) != hipSuccess)
      return GKV_ERR_HIP;
    if (pool->d_ring_table &&
        hipMemcpyAsync(pool->d_ring_table, pool->h_ring_table.data(),
                       pool->h_ring_table.size() * 4, hipMemcpyHostToDevice, s) != hipSuccess)
      return GKV_ERR_HIP;
    if (hipStreamSynchronize(s) != hipSuccess)
      return GKV_ERR_HIP;
    pool->whole = false;
    pool->pending.clear();
    return GKV_OK;
  }
  if (pool->pending.empty())
    return GKV_OK;
  // One pair per changed entry, its latest value (a reserve after a free of
  // the same entry within one sync leaves two pairs; the host table holds
  // the value that counts).
  std::vector<int2> &pend = pool->pending;
  std::sort(pend.begin(), pend.end(), [](const int2 &x, const int2 &y) { return x.x < y.x; });
  pend.erase(std::unique(pend.begin(), pend.end(),
                         [](const int2 &x, const int2 &y) { return x.x == y.x; }),
             pend.end());
  for (int2 &e : pend)
    e.y = pool->h_table[e.x];
  const size_t n = pend.size();
  if (n > pool->stage_cap) {
    pool->free_stage();
    const size_t cap = std::max<size_t>(n, 4096);
    for (int i = 0; i < 2; i++)
      if (hipHostMalloc((void **)&pool->h_stage[i], cap * sizeof(int2), hipHostMallocDefault) !=
              hipSuccess ||
          hipMalloc((void **)&pool->d_stage[i], cap * sizeof(int2)) != hipSuccess ||
          hipEventCreateWithFlags(&pool->stage_done[i], hipEventDisableTiming) != hipSuccess) {
        pool->free_stage();
        return GKV_ERR_HIP;
      }
    pool->stage_cap = cap;
  }
  const int k = pool->stage_i;
  // the staging buffer's previous copy (two syncs ago) has long completed
  // in practice; the wait only guards the case where it has not
  if (hipEventSynchronize(pool->stage_done[k]) != hipSuccess)
    return GKV_ERR_HIP;
  std::memcpy(pool->h_stage[k], pend.data(), n * sizeof(int2));
  if (hipMemcpyAsync(pool->d_stage[k], pool->h_stage[k], n * sizeof(int2), hipMemcpyHostToDevice,
                     s) != hipSuccess)
    return GKV_ERR_HIP;
  hipLaunchKernelGGL(pool_scatter_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     pool->d_table, pool->d_stage[k], (int)n);
  if (hipGetLastError() != hipSuccess || hipEventRecord(pool->stage_done[k], s) != hipSuccess)
    return GKV_ERR_HIP;
  pool->stage_i ^= 1;
  pend.clear();
  return GKV_OK;
}

extern "C" int gkv_pool_layer_view_from(const gkv_pool *pool, int32_t layer, int32_t first_seq,
                                        gkv_cache_view *view) {
  if (!pool || !view || layer < 0 || layer >= pool->cfg.n_layers || first_seq < 0 ||
      first_seq >= pool->cfg.max_seqs)
    return GKV_ERR_ARG;
  const int i = pool->layer_index[layer];
  gkv_cache_view v{};
  v.n_kv_heads = pool->cfg.n_kv_heads;
  v.v_format = pool->cfg.v_format;
  if (pool->layer_is_window[layer]) {
    v.k = pool->k_ring[i];
    v.v = pool->v_ring[i];
    v.v_scale = pool->s_ring[i];
    v.block_table = pool->d_ring_table + (size_t)first_seq * pool->ring_blocks;
    v.table_stride = pool->ring_blocks;
    v.num_blocks = (int32_t)pool->num_ring_blocks;
    v.ring = pool->cfg.window;
  } else {
    v.k = pool->k_full[i];
    v.v = pool->v_full[i];
    v.v_scale = pool->s_full[i];
    v.block_table = pool->d_table + (size_t)first_seq * pool->table_stride;
    v.table_stride = pool->table_stride;
    v.num_blocks = (int32_t)pool->num_blocks;
    v.ring = 0;
  }
  *view = v;
  return GKV_OK;
}

extern "C" int gkv_pool_layer_view(const gkv_pool *pool, int32_t layer, gkv_cache_view *view) {
  return gkv_pool_layer_view_from(pool, layer, 0, view);
}

extern "C" int64_t gkv_pool_free_blocks(const gkv_pool *pool) {
  return pool ? (int64_t)pool->free_blocks.size() : -1;
}

extern "C" int64_t gkv_pool_num_blocks(const gkv_pool *pool) {
  return pool ? pool->num_blocks : -1;
}

extern "C" int64_t gkv_pool_device_bytes(const gkv_pool *pool) {
  return pool ? pool->device_bytes : -1;
}

extern "C" int gkv_pool_seq_blocks(const gkv_pool *pool, int32_t seq_id, int32_t *blocks,
                                   int32_t n, int32_t *n_used) {
  if (!pool || n < 0 || (n > 0 && !blocks))
    return GKV_ERR_ARG;
  if (seq_id < 0 || seq_id >= pool->cfg.max_seqs || !pool->seq_live[seq_id])
    return GKV_ERR_BLOCK;
  const int32_t used = pool->seq_blocks[seq_id];
  const int32_t *row = &pool->h_table[(size_t)seq_id * pool->table_stride];
  for (int32_t j = 0; j < std::min(n, used); j++)
    blocks[j] = row[j];
  if (n_used)
    *n_used = used;
  return GKV_OK;
}
