// pool.cpp — error plumbing and the paged-pool free list behind the C ABI.
//
// Mirrors TheRadDani/memopt-transformer-runtime src/csrc/kv_cache.cu:83-201
// (KVCachePool singleton, FIFO free list under a mutex, allocate_block
// returning -1 when exhausted) with two deliberate differences:
//   * storage is allocated and owned by the caller and registered here;
//   * invalid init parameters tear the previous pool down (the reference
//     throws after its idempotency check and leaves the old pool live).
#include <deque>
#include <mutex>
#include <string>

#include "common.hpp"

namespace memopt {

static thread_local std::string t_last_error;

void set_error(const std::string &msg) { t_last_error = msg; }
void clear_error() { t_last_error.clear(); }

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": kernel launch failed: " + hipGetErrorString(e));
    return MEMOPT_ERR_HIP;
  }
  return MEMOPT_OK;
}

namespace {
struct Pool {
  std::mutex mu;
  PoolView view;
  std::deque<int64_t> free_list;  // FIFO, as std::queue in the reference
};
Pool g_pool;
}  // namespace

PoolView pool_snapshot() {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  return g_pool.view;
}

}  // namespace memopt

using namespace memopt;

extern "C" {

const char *memopt_last_error(void) { return t_last_error.c_str(); }

const char *memopt_get_hello(void) {
  return "MemOpt C++ Backend Initialized (HIP, gfx950 INT4 KV-cache data plane)";
}

int memopt_init_pool(int64_t num_blocks, int32_t block_size, int32_t num_heads,
                     int32_t head_dim, int32_t kv_format, void *key_pool,
                     void *value_pool, void *key_scales, void *value_scales) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  // Tear down first: a failed init leaves no pool behind.
  g_pool.view = PoolView();
  g_pool.free_list.clear();
  MEMOPT_REQUIRE(num_blocks > 0, MEMOPT_ERR_INVALID, "init_pool: num_blocks must be > 0");
  MEMOPT_REQUIRE(block_size > 0, MEMOPT_ERR_INVALID, "init_pool: block_size must be > 0");
  MEMOPT_REQUIRE(num_heads > 0, MEMOPT_ERR_INVALID, "init_pool: num_heads must be > 0");
  MEMOPT_REQUIRE(head_dim > 0, MEMOPT_ERR_INVALID, "init_pool: head_dim must be > 0");
  MEMOPT_REQUIRE(head_dim % 2 == 0, MEMOPT_ERR_INVALID,
                 "init_pool: head_dim must be even for fp16 coalesced access");
  MEMOPT_REQUIRE(kv_format == MEMOPT_KV_FP16 || kv_format == MEMOPT_KV_INT4,
                 MEMOPT_ERR_INVALID, "init_pool: unknown kv_format");
  if (kv_format == MEMOPT_KV_INT4) {
    MEMOPT_REQUIRE(head_dim % 64 == 0, MEMOPT_ERR_INVALID,
                   "init_pool: INT4 pools need head_dim % 64 == 0 (group size 64)");
    MEMOPT_REQUIRE(block_size == 16, MEMOPT_ERR_INVALID, "init_pool: INT4 pools use 16-token pages");
    MEMOPT_REQUIRE(key_pool, MEMOPT_ERR_INVALID, "init_pool: null page buffer");
    value_pool = key_scales = value_scales = nullptr;
  } else {
    MEMOPT_REQUIRE(key_pool && value_pool, MEMOPT_ERR_INVALID, "init_pool: null pool storage");
  }
  PoolView v;
  v.initialized = true;
  v.num_blocks = num_blocks;
  v.block_size = block_size;
  v.num_heads = num_heads;
  v.head_dim = head_dim;
  v.kv_format = kv_format;
  v.key = key_pool;
  v.value = value_pool;
  v.key_scales = key_scales;
  v.value_scales = value_scales;
  g_pool.view = v;
  for (int64_t i = 0; i < num_blocks; ++i) g_pool.free_list.push_back(i);
  return MEMOPT_OK;
}

int memopt_pool_set_storage(int32_t kv_format, void *key_pool, void *value_pool) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  PoolView &v = g_pool.view;
  MEMOPT_REQUIRE(v.initialized, MEMOPT_ERR_STATE, "pool_set_storage: pool not initialized");
  MEMOPT_REQUIRE(kv_format == MEMOPT_KV_FP16 || kv_format == MEMOPT_KV_INT4, MEMOPT_ERR_INVALID,
                 "pool_set_storage: unknown kv_format");
  if (kv_format == MEMOPT_KV_INT4) {
    MEMOPT_REQUIRE(v.head_dim % 64 == 0 && v.block_size == 16, MEMOPT_ERR_INVALID,
                   "pool_set_storage: INT4 pools need 16-token pages and head_dim % 64 == 0");
    MEMOPT_REQUIRE(key_pool, MEMOPT_ERR_INVALID, "pool_set_storage: null page buffer");
    value_pool = nullptr;
  } else {
    MEMOPT_REQUIRE(key_pool && value_pool, MEMOPT_ERR_INVALID, "pool_set_storage: null pool storage");
  }
  v.kv_format = kv_format;
  v.key = key_pool;
  v.value = value_pool;
  v.key_scales = v.value_scales = nullptr;
  return MEMOPT_OK;
}

int memopt_pool_info(int64_t *num_blocks, int32_t *block_size, int32_t *num_heads,
                     int32_t *head_dim, int32_t *kv_format) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  if (!g_pool.view.initialized) return 0;
  if (num_blocks) *num_blocks = g_pool.view.num_blocks;
  if (block_size) *block_size = g_pool.view.block_size;
  if (num_heads) *num_heads = g_pool.view.num_heads;
  if (head_dim) *head_dim = g_pool.view.head_dim;
  if (kv_format) *kv_format = g_pool.view.kv_format;
  return 1;
}

int memopt_reset_pool(void) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  g_pool.view = PoolView();
  g_pool.free_list.clear();
  return MEMOPT_OK;
}

int memopt_allocate_block(int64_t *block_idx) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  MEMOPT_REQUIRE(g_pool.view.initialized, MEMOPT_ERR_STATE, "allocate_block: pool not initialized");
  if (g_pool.free_list.empty()) {
    *block_idx = -1;  // exhausted: the caller must evict or fail
    return MEMOPT_OK;
  }
  *block_idx = g_pool.free_list.front();
  g_pool.free_list.pop_front();
  return MEMOPT_OK;
}

int memopt_free_block(int64_t block_idx) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  MEMOPT_REQUIRE(g_pool.view.initialized, MEMOPT_ERR_STATE, "free_block: pool not initialized");
  MEMOPT_REQUIRE(block_idx >= 0 && block_idx < g_pool.view.num_blocks, MEMOPT_ERR_INVALID,
                 "free_block: block_idx out of range");
  g_pool.free_list.push_back(block_idx);
  return MEMOPT_OK;
}

int memopt_free_blocks_count(int64_t *count) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  *count = (int64_t)g_pool.free_list.size();
  return MEMOPT_OK;
}

}  // extern "C"
