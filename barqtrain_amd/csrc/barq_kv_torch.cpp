// barqtrain_cuda: the PyTorch-ROCm extension module the BarqTrain loader imports
// (python/barqtrain/_ffi.py:117-121).  It only checks tensors and forwards raw pointers, sizes
// and the current HIP stream to the C ABI of libbarq_kv.so (include/barq_kv.h); every kernel
// lives there.  Host-only C++: no device code is compiled into this module.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <string>
#include <tuple>
#include <vector>

#include "barq_kv.h"

namespace {

void* current_stream(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

void check_status(int rc, const char* what) {
  TORCH_CHECK(rc == BARQ_KV_OK, what, ": ", barq_kv_status_string(rc));
}

int64_t elem_bytes_of(const at::Tensor& t) { return (int64_t)t.element_size(); }

// Same shape, and the same strides along every dimension of size > 1 (a size-1 dimension's
// stride never enters an address).  HF decode steps hand over K and V that differ only in the
// stride of their size-1 sequence dimension.
bool same_layout(const at::Tensor& a, const at::Tensor& b) {
  if (a.sizes() != b.sizes()) return false;
  for (int64_t d = 0; d < a.dim(); ++d)
    if (a.size(d) > 1 && a.stride(d) != b.stride(d)) return false;
  return true;
}

// The pool is passed as (key_pages, value_pages, block_table, seq_lens, high_water, free_pages,
// ctrl, page_shares), the tensors of barqtrain_amd.paged.PagePool.
barq_kv_pool pool_from(const std::vector<at::Tensor>& t) {
  TORCH_CHECK(t.size() == 8, "a page pool is 8 tensors");
  const at::Tensor& kp = t[0];
  const at::Tensor& vp = t[1];
  TORCH_CHECK(kp.is_cuda() && vp.is_cuda(), "page pool must live on a GPU");
  TORCH_CHECK(kp.dim() == 4 && vp.sizes() == kp.sizes(),
              "key/value pages must be [num_pages, page_size, kv_heads, head_dim]");
  TORCH_CHECK(kp.is_contiguous() && vp.is_contiguous(), "pages must be contiguous");
  TORCH_CHECK(kp.scalar_type() == vp.scalar_type(), "key/value pages must share dtype");
  for (size_t i = 2; i < 8; ++i) {
    TORCH_CHECK(t[i].scalar_type() == at::kInt && t[i].is_contiguous() && t[i].is_cuda() &&
                    t[i].get_device() == kp.get_device(),
                "page-pool metadata must be contiguous int32 on the pool's device");
  }
  TORCH_CHECK(t[2].dim() == 2, "block_table must be [max_batch, max_blocks]");
  barq_kv_pool p;
  p.key_pages = kp.data_ptr();
  p.value_pages = vp.data_ptr();
  p.block_table = t[2].data_ptr<int32_t>();
  p.seq_lens = t[3].data_ptr<int32_t>();
  p.high_water = t[4].data_ptr<int32_t>();
  p.free_pages = t[5].data_ptr<int32_t>();
  p.ctrl = t[6].data_ptr<int32_t>();
  p.page_shares = t[7].data_ptr<int32_t>();
  p.num_pages = kp.size(0);
  p.page_size = kp.size(1);
  p.kv_heads = kp.size(2);
  p.head_dim = kp.size(3);
  p.elem_bytes = elem_bytes_of(kp);
  p.max_batch = t[2].size(0);
  p.max_blocks = t[2].size(1);
  TORCH_CHECK(t[3].numel() == p.max_batch && t[4].numel() == p.max_batch, "row metadata size mismatch");
  TORCH_CHECK(t[5].numel() == p.num_pages, "free_pages must hold num_pages entries");
  TORCH_CHECK(t[6].numel() == BARQ_KV_CTRL_WORDS, "ctrl must hold BARQ_KV_CTRL_WORDS entries");
  TORCH_CHECK(t[7].numel() == p.num_pages, "page_shares must hold num_pages entries");
  return p;
}

void check_states(const barq_kv_pool& p, const at::Tensor& pages, const at::Tensor& k,
                  const at::Tensor& v) {
  TORCH_CHECK(k.is_cuda() && v.is_cuda() && k.get_device() == pages.get_device(),
              "key_states and value_states must stay on the cache device");
  TORCH_CHECK(k.dim() == 4 && v.sizes() == k.sizes(), "key_states and value_states must have identical shapes");
  TORCH_CHECK(k.scalar_type() == pages.scalar_type() && v.scalar_type() == pages.scalar_type(),
              "key_states and value_states must stay in the cache dtype");
  TORCH_CHECK(k.size(1) == p.kv_heads && k.size(3) == p.head_dim, "key_states kv_heads/head_dim mismatch");
  TORCH_CHECK(k.stride(3) == 1 && v.stride(3) == 1, "head_dim of the states must be contiguous");
  TORCH_CHECK(same_layout(k, v), "key_states and value_states must share strides");
}

void check_out(const barq_kv_pool& p, const at::Tensor& pages, const at::Tensor& ko,
               const at::Tensor& vo, int64_t batch, int64_t seq_out) {
  TORCH_CHECK(ko.is_cuda() && vo.is_cuda() && ko.get_device() == pages.get_device(),
              "outputs must be on the cache device");
  TORCH_CHECK(ko.dim() == 4 && same_layout(ko, vo),
              "outputs must be [batch, kv_heads, seq, head_dim] with equal strides");
  TORCH_CHECK(ko.scalar_type() == pages.scalar_type() && vo.scalar_type() == pages.scalar_type(),
              "outputs must have the cache dtype");
  TORCH_CHECK(ko.size(0) >= batch && ko.size(1) == p.kv_heads && ko.size(2) >= seq_out &&
                  ko.size(3) == p.head_dim,
              "outputs too small for [batch, kv_heads, seq_out, head_dim]");
  TORCH_CHECK(ko.stride(3) == 1, "head_dim of the outputs must be contiguous");
}

// Reference binding: barqtrain_cuda.paged_kv_append_ (csrc/src/bindings.cpp:43-49,74-75) with
// the checks and messages of paged_kv_append_cuda (csrc/kernels/paged_kv_cache.cu:64-99,127).
void paged_kv_append_(at::Tensor key_cache, at::Tensor value_cache, at::Tensor seq_lens,
                      at::Tensor key_states, at::Tensor value_states) {
  TORCH_CHECK(key_cache.is_cuda(), "key_cache must be a CUDA tensor");
  TORCH_CHECK(value_cache.is_cuda(), "value_cache must be a CUDA tensor");
  TORCH_CHECK(seq_lens.is_cuda(), "seq_lens must be a CUDA tensor");
  TORCH_CHECK(key_states.is_cuda(), "key_states must be a CUDA tensor");
  TORCH_CHECK(value_states.is_cuda(), "value_states must be a CUDA tensor");
  TORCH_CHECK(key_cache.dim() == 5, "key_cache must have shape [batch, kv_heads, max_blocks, page_size, head_dim]");
  TORCH_CHECK(value_cache.sizes() == key_cache.sizes(), "value_cache must match key_cache");
  TORCH_CHECK(seq_lens.dim() == 1, "seq_lens must have shape [batch]");
  TORCH_CHECK(key_states.dim() == 4, "key_states must have shape [batch, kv_heads, seq, head_dim]");
  TORCH_CHECK(value_states.sizes() == key_states.sizes(), "value_states must match key_states");
  TORCH_CHECK(key_cache.scalar_type() == key_states.scalar_type(), "key_cache and key_states must share dtype");
  TORCH_CHECK(value_cache.scalar_type() == value_states.scalar_type(), "value_cache and value_states must share dtype");
  TORCH_CHECK(key_cache.is_contiguous(), "key_cache must be contiguous");
  TORCH_CHECK(value_cache.is_contiguous(), "value_cache must be contiguous");
  TORCH_CHECK(key_cache.scalar_type() == value_cache.scalar_type(), "key_cache and value_cache must share dtype");

  const int64_t batch = key_states.size(0);
  const int64_t heads = key_states.size(1);
  const int64_t tokens = key_states.size(2);
  const int64_t head_dim = key_states.size(3);
  const int64_t max_blocks = key_cache.size(2);
  const int64_t page_size = key_cache.size(3);
  const int64_t max_cache_len = max_blocks * page_size;
  TORCH_CHECK(batch <= key_cache.size(0), "key_cache batch dimension is too small");
  TORCH_CHECK(heads == key_cache.size(1), "key_cache kv_heads dimension does not match key_states");
  TORCH_CHECK(head_dim == key_cache.size(4), "key_cache head_dim dimension does not match key_states");
  TORCH_CHECK(batch <= seq_lens.size(0), "seq_lens batch dimension is too small");
  if (batch == 0) return;

  c10::DeviceGuard guard(key_cache.device());
  at::Tensor lens32 = seq_lens.to(at::kInt).contiguous();
  // The capacity check needs the lengths on the host, as the reference's does (:93).
  const int64_t max_start = lens32.narrow(0, 0, batch).max().item<int32_t>();
  TORCH_CHECK(max_start + tokens <= max_cache_len, "paged KV cache capacity exceeded: requested ",
              max_start + tokens, " tokens, max_cache_len=", max_cache_len);

  at::Tensor ks = key_states.stride(3) == 1 ? key_states : key_states.contiguous();
  at::Tensor vs = value_states.stride(3) == 1 ? value_states : value_states.contiguous();
  if (!same_layout(ks, vs)) {
    ks = ks.contiguous();
    vs = vs.contiguous();
  }
  const bool same = lens32.data_ptr() == seq_lens.data_ptr();
  const int rc = barq_kv_append_dense(key_cache.data_ptr(), value_cache.data_ptr(), lens32.data_ptr<int32_t>(),
                                      ks.data_ptr(), vs.data_ptr(), batch, heads, tokens, head_dim,
                                      key_cache.size(0), max_blocks, page_size, elem_bytes_of(key_cache),
                                      ks.stride(0), ks.stride(1), ks.stride(2), current_stream(key_cache));
  check_status(rc, "paged_kv_append_");
  if (!same) seq_lens.narrow(0, 0, batch).add_(tokens);  // lens32 was a converted copy
}

void pool_reset_(std::vector<at::Tensor> pool, c10::optional<at::Tensor> page_order) {
  barq_kv_pool p = pool_from(pool);
  c10::DeviceGuard guard(pool[0].device());
  const int32_t* order = nullptr;
  if (page_order.has_value() && page_order->defined()) {
    const at::Tensor& o = *page_order;
    TORCH_CHECK(o.is_cuda() && o.scalar_type() == at::kInt && o.is_contiguous() && o.numel() == p.num_pages,
                "page_order must be a contiguous int32 permutation of the pages on the pool's device");
    order = o.data_ptr<int32_t>();
  }
  check_status(barq_kv_pool_reset(&p, order, current_stream(pool[0])), "pool_reset_");
}

void pool_append_(std::vector<at::Tensor> pool, at::Tensor key_states, at::Tensor value_states) {
  barq_kv_pool p = pool_from(pool);
  check_states(p, pool[0], key_states, value_states);
  c10::DeviceGuard guard(pool[0].device());
  const int rc = barq_kv_append(&p, key_states.data_ptr(), value_states.data_ptr(), key_states.size(0),
                                key_states.size(2), key_states.stride(0), key_states.stride(1),
                                key_states.stride(2), current_stream(pool[0]));
  check_status(rc, "pool_append_");
}

void pool_gather(std::vector<at::Tensor> pool, at::Tensor key_out, at::Tensor value_out,
                 int64_t batch, int64_t seq_out, int64_t flags) {
  barq_kv_pool p = pool_from(pool);
  check_out(p, pool[0], key_out, value_out, batch, seq_out);
  c10::DeviceGuard guard(pool[0].device());
  const int rc = barq_kv_gather(&p, key_out.data_ptr(), value_out.data_ptr(), batch, seq_out,
                                key_out.stride(0), key_out.stride(1), key_out.stride(2), flags,
                                current_stream(pool[0]));
  check_status(rc, "pool_gather");
}

void pool_update_(std::vector<at::Tensor> pool, at::Tensor key_states, at::Tensor value_states,
                  at::Tensor key_out, at::Tensor value_out, int64_t seq_out, int64_t flags) {
  barq_kv_pool p = pool_from(pool);
  check_states(p, pool[0], key_states, value_states);
  const int64_t batch = key_states.size(0);
  check_out(p, pool[0], key_out, value_out, batch, seq_out);
  c10::DeviceGuard guard(pool[0].device());
  const int rc = barq_kv_update(&p, key_states.data_ptr(), value_states.data_ptr(), batch,
                                key_states.size(2), key_states.stride(0), key_states.stride(1),
                                key_states.stride(2), key_out.data_ptr(), value_out.data_ptr(), seq_out,
                                key_out.stride(0), key_out.stride(1), key_out.stride(2), flags,
                                current_stream(pool[0]));
  check_status(rc, "pool_update_");
}

void pool_crop_(std::vector<at::Tensor> pool, int64_t batch, int64_t max_length) {
  barq_kv_pool p = pool_from(pool);
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_crop(&p, batch, max_length, current_stream(pool[0])), "pool_crop_");
}

void pool_free_rows_(std::vector<at::Tensor> pool, at::Tensor rows) {
  barq_kv_pool p = pool_from(pool);
  TORCH_CHECK(rows.is_cuda() && rows.scalar_type() == at::kInt && rows.is_contiguous() &&
                  rows.get_device() == pool[0].get_device(),
              "rows must be contiguous int32 on the pool's device");
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_free_rows(&p, rows.data_ptr<int32_t>(), rows.numel(), current_stream(pool[0])),
               "pool_free_rows_");
}

void pool_copy_rows_(std::vector<at::Tensor> src, std::vector<at::Tensor> dst, at::Tensor rows) {
  barq_kv_pool ps = pool_from(src);
  barq_kv_pool pd = pool_from(dst);
  TORCH_CHECK(src[0].scalar_type() == dst[0].scalar_type(), "pools must share dtype");
  TORCH_CHECK(src[0].get_device() == dst[0].get_device(), "pools must share a device");
  TORCH_CHECK(rows.is_cuda() && rows.scalar_type() == at::kInt && rows.is_contiguous() &&
                  rows.get_device() == src[0].get_device(),
              "rows must be contiguous int32 on the pool's device");
  c10::DeviceGuard guard(src[0].device());
  check_status(barq_kv_copy_rows(&ps, &pd, rows.data_ptr<int32_t>(), rows.numel(), current_stream(src[0])),
               "pool_copy_rows_");
}

void pool_select_rows_(std::vector<at::Tensor> pool, at::Tensor rows, at::Tensor workspace) {
  barq_kv_pool p = pool_from(pool);
  TORCH_CHECK(rows.is_cuda() && rows.scalar_type() == at::kInt && rows.is_contiguous() &&
                  rows.get_device() == pool[0].get_device(),
              "rows must be contiguous int32 on the pool's device");
  TORCH_CHECK(workspace.is_cuda() && workspace.scalar_type() == at::kInt && workspace.is_contiguous() &&
                  workspace.get_device() == pool[0].get_device(),
              "workspace must be contiguous int32 on the pool's device");
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_select_rows(&p, rows.data_ptr<int32_t>(), rows.numel(), workspace.data_ptr<int32_t>(),
                                   workspace.numel(), current_stream(pool[0])),
               "pool_select_rows_");
}

// A pool's fp8 cold store as (key_codes, value_codes, key_scales, value_scales, free_cold,
// cold_shares), the tensors of barqtrain_amd.paged.QuantPagePool, and its residual window.
barq_kv_cold cold_from(const barq_kv_pool& p, const at::Tensor& pages, const std::vector<at::Tensor>& t,
                       int64_t window) {
  TORCH_CHECK(t.size() == 6, "a cold store is 6 tensors");
  for (size_t i = 0; i < 6; ++i)
    TORCH_CHECK(t[i].is_cuda() && t[i].is_contiguous() && t[i].get_device() == pages.get_device() &&
                    t[i].scalar_type() == (i < 4 ? at::kByte : at::kInt),
                "cold-store tensors must be contiguous (uint8 codes and scales, int32 free list and shares) on the "
                "pool's device");
  const int64_t n = t[0].size(0);
  TORCH_CHECK(t[0].dim() == 4 && t[0].size(1) == p.page_size && t[0].size(2) == p.kv_heads &&
                  t[0].size(3) == p.head_dim && t[1].sizes() == t[0].sizes(),
              "codes must be [num_cold, page_size, kv_heads, head_dim]");
  TORCH_CHECK(t[2].numel() == n * p.kv_heads * p.head_dim && t[3].numel() == n * p.page_size * p.kv_heads &&
                  t[4].numel() == n && t[5].numel() == n,
              "cold-store scale / free-list / shares sizes do not match num_cold");
  barq_kv_cold c;
  c.key_codes = t[0].data_ptr();
  c.value_codes = t[1].data_ptr();
  c.key_scales = t[2].data_ptr();
  c.value_scales = t[3].data_ptr();
  c.free_cold = t[4].data_ptr<int32_t>();
  c.cold_shares = t[5].data_ptr<int32_t>();
  c.num_cold = n;
  c.window = window;
  const auto dt = pages.scalar_type();
  TORCH_CHECK(dt == at::kBFloat16 || dt == at::kHalf || dt == at::kFloat,
              "quantised pages need a bfloat16, float16 or float32 cache");
  c.element_type = dt == at::kBFloat16 ? BARQ_KV_BF16 : dt == at::kHalf ? BARQ_KV_FP16 : BARQ_KV_FP32;
  return c;
}

void pool_cold_reset_(std::vector<at::Tensor> pool, std::vector<at::Tensor> cold, int64_t window) {
  barq_kv_pool p = pool_from(pool);
  barq_kv_cold c = cold_from(p, pool[0], cold, window);
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_cold_reset(&p, &c, current_stream(pool[0])), "pool_cold_reset_");
}

void pool_compress_(std::vector<at::Tensor> pool, std::vector<at::Tensor> cold, int64_t window, int64_t batch) {
  barq_kv_pool p = pool_from(pool);
  barq_kv_cold c = cold_from(p, pool[0], cold, window);
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_compress(&p, &c, batch, current_stream(pool[0])), "pool_compress_");
}

void pool_gather_cold(std::vector<at::Tensor> pool, std::vector<at::Tensor> cold, int64_t window,
                      at::Tensor key_out, at::Tensor value_out, int64_t batch, int64_t seq_out, int64_t flags) {
  barq_kv_pool p = pool_from(pool);
  barq_kv_cold c = cold_from(p, pool[0], cold, window);
  check_out(p, pool[0], key_out, value_out, batch, seq_out);
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_gather_cold(&p, &c, key_out.data_ptr(), value_out.data_ptr(), batch, seq_out,
                                   key_out.stride(0), key_out.stride(1), key_out.stride(2), flags,
                                   current_stream(pool[0])),
               "pool_gather_cold");
}

void pool_update_cold_(std::vector<at::Tensor> pool, std::vector<at::Tensor> cold, int64_t window,
                       at::Tensor key_states, at::Tensor value_states, at::Tensor key_out, at::Tensor value_out,
                       int64_t seq_out, int64_t flags) {
  barq_kv_pool p = pool_from(pool);
  barq_kv_cold c = cold_from(p, pool[0], cold, window);
  check_states(p, pool[0], key_states, value_states);
  const int64_t batch = key_states.size(0);
  check_out(p, pool[0], key_out, value_out, batch, seq_out);
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_update_cold(&p, &c, key_states.data_ptr(), value_states.data_ptr(), batch,
                                   key_states.size(2), key_states.stride(0), key_states.stride(1),
                                   key_states.stride(2), key_out.data_ptr(), value_out.data_ptr(), seq_out,
                                   key_out.stride(0), key_out.stride(1), key_out.stride(2), flags,
                                   current_stream(pool[0])),
               "pool_update_cold_");
}

void pool_free_rows_cold_(std::vector<at::Tensor> pool, std::vector<at::Tensor> cold, int64_t window,
                          at::Tensor rows) {
  barq_kv_pool p = pool_from(pool);
  barq_kv_cold c = cold_from(p, pool[0], cold, window);
  TORCH_CHECK(rows.is_cuda() && rows.scalar_type() == at::kInt && rows.is_contiguous() &&
                  rows.get_device() == pool[0].get_device(),
              "rows must be contiguous int32 on the pool's device");
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_free_rows_cold(&p, &c, rows.data_ptr<int32_t>(), rows.numel(), current_stream(pool[0])),
               "pool_free_rows_cold_");
}

void pool_crop_cold_(std::vector<at::Tensor> pool, std::vector<at::Tensor> cold, int64_t window, int64_t batch,
                     int64_t max_length) {
  barq_kv_pool p = pool_from(pool);
  barq_kv_cold c = cold_from(p, pool[0], cold, window);
  c10::DeviceGuard guard(pool[0].device());
  check_status(barq_kv_crop_cold(&p, &c, batch, max_length, current_stream(pool[0])), "pool_crop_cold_");
}

// One selection applied to pools with cold stores (a model's layers): pools[i] with colds[i].
void pool_select_rows_cold_(std::vector<std::vector<at::Tensor>> pools, std::vector<std::vector<at::Tensor>> colds,
                            int64_t window, at::Tensor rows, at::Tensor workspace) {
  TORCH_CHECK(!pools.empty() && pools.size() == colds.size(), "one cold store per pool");
  std::vector<barq_kv_pool> ps;
  std::vector<barq_kv_cold> cs;
  for (size_t i = 0; i < pools.size(); ++i) {
    ps.push_back(pool_from(pools[i]));
    cs.push_back(cold_from(ps.back(), pools[i][0], colds[i], window));
    TORCH_CHECK(pools[i][0].get_device() == rows.get_device(), "the pools and rows must share a device");
  }
  TORCH_CHECK(rows.is_cuda() && rows.scalar_type() == at::kInt && rows.is_contiguous(),
              "rows must be contiguous int32 on the pools' device");
  TORCH_CHECK(workspace.is_cuda() && workspace.scalar_type() == at::kInt && workspace.is_contiguous() &&
                  workspace.get_device() == rows.get_device(),
              "workspace must be contiguous int32 on the pools' device");
  c10::DeviceGuard guard(rows.device());
  check_status(barq_kv_select_rows_cold_layers(ps.data(), cs.data(), (int64_t)ps.size(), rows.data_ptr<int32_t>(),
                                               rows.numel(), workspace.data_ptr<int32_t>(), workspace.numel(),
                                               current_stream(rows)),
               "pool_select_rows_cold_");
}

// One decode-step call of PagePool.update / append with its host planning in C++: the capacity
// and free-page checks of the host shadow (int64 arrays lens / hw, updated in place on success),
// output allocation and the launch.  handle: pool_group of this one pool; pages: its key_pages
// (device, dtype).  Returns (key_out, value_out, pages taken); pages taken < 0 when the call must
// take the checked Python path instead, which raises the exact error (-1: capacity exceeded, -2:
// not enough free pages by the host count, -3: nothing to append, -4: states the pool cannot
// take as they are).
std::tuple<at::Tensor, at::Tensor, int64_t> pool_step_(at::Tensor handle, at::Tensor pages, at::Tensor key_states,
                                                       at::Tensor value_states, py::buffer lens, py::buffer hw,
                                                       int64_t free_count, bool free_exact, int64_t limit,
                                                       int64_t flags, bool gather) {
  TORCH_CHECK(handle.device().is_cpu() && handle.scalar_type() == at::kByte &&
                  handle.numel() == (int64_t)sizeof(barq_kv_pool),
              "not a one-pool group (see pool_group)");
  const barq_kv_pool p = *reinterpret_cast<const barq_kv_pool*>(handle.data_ptr<uint8_t>());
  TORCH_CHECK(pages.is_cuda() && pages.data_ptr() == p.key_pages, "pages do not belong to the handle");
  at::Tensor none;
  if (key_states.dim() != 4 || value_states.sizes() != key_states.sizes() || key_states.size(1) != p.kv_heads ||
      key_states.size(3) != p.head_dim || !key_states.is_cuda() || !value_states.is_cuda() ||
      key_states.get_device() != pages.get_device() || value_states.get_device() != pages.get_device() ||
      key_states.scalar_type() != pages.scalar_type() || value_states.scalar_type() != pages.scalar_type() ||
      key_states.size(0) > p.max_batch)
    return {none, none, -4};
  const int64_t batch = key_states.size(0), tokens = key_states.size(2);
  const py::buffer_info li = lens.request(true), hi = hw.request(true);
  TORCH_CHECK(li.itemsize == 8 && hi.itemsize == 8 && li.ndim == 1 && hi.ndim == 1 && li.shape[0] >= batch &&
                  hi.shape[0] >= batch && li.strides[0] == 8 && hi.strides[0] == 8,
              "lens / hw must be contiguous int64 arrays of at least batch entries");
  int64_t* L = static_cast<int64_t*>(li.ptr);
  int64_t* W = static_cast<int64_t*>(hi.ptr);
  if (batch == 0 || tokens == 0) return {none, none, -3};
  const int64_t P = p.page_size;
  int64_t worst = 0, need = 0;
  for (int64_t r = 0; r < batch; ++r) {
    const int64_t end = L[r] + tokens;
    worst = std::max(worst, end);
    need += std::max<int64_t>(std::min((end + P - 1) / P, p.max_blocks) - (W[r] + P - 1) / P, 0);
  }
  if (worst > limit || worst > p.max_blocks * P) return {none, none, -1};
  if (need > free_count) return {none, none, -2};
  at::Tensor k = key_states, v = value_states;
  if (k.stride(3) != 1 || v.stride(3) != 1 || !same_layout(k, v)) {
    k = k.contiguous();
    v = v.contiguous();
  }
  c10::DeviceGuard guard(pages.device());
  at::Tensor ko, vo;
  int rc;
  if (gather) {
    at::Tensor both = at::empty({2, batch, p.kv_heads, worst, p.head_dim}, pages.options());
    ko = both[0];
    vo = both[1];
    if (flags == 0 && free_exact && batch <= 64) {
      // The shadow is exact: the launch takes the row state in its arguments.
      int32_t l32[64], w32[64];
      for (int64_t r = 0; r < batch; ++r) {
        l32[r] = (int32_t)L[r];
        w32[r] = (int32_t)W[r];
      }
      rc = barq_kv_update_known(&p, k.data_ptr(), v.data_ptr(), batch, tokens, k.stride(0), k.stride(1),
                                k.stride(2), ko.data_ptr(), vo.data_ptr(), worst, ko.stride(0), ko.stride(1),
                                ko.stride(2), l32, w32, free_count, current_stream(pages));
    } else {
      rc = barq_kv_update(&p, k.data_ptr(), v.data_ptr(), batch, tokens, k.stride(0), k.stride(1), k.stride(2),
                          ko.data_ptr(), vo.data_ptr(), worst, ko.stride(0), ko.stride(1), ko.stride(2), flags,
                          current_stream(pages));
    }
  } else {
    rc = barq_kv_append(&p, k.data_ptr(), v.data_ptr(), batch, tokens, k.stride(0), k.stride(1), k.stride(2),
                        current_stream(pages));
  }
  check_status(rc, gather ? "pool_update_" : "pool_append_");
  for (int64_t r = 0; r < batch; ++r) {
    L[r] += tokens;
    W[r] = std::max(W[r], L[r]);
  }
  return {ko, vo, need};
}

// The pools of a model's layers packed as an array of barq_kv_pool (a CPU uint8 tensor), for
// the batched entry points.  The array holds raw device pointers: the caller keeps the pools'
// tensors alive and unmoved while it uses it.
at::Tensor pool_group(std::vector<std::vector<at::Tensor>> pools) {
  TORCH_CHECK(!pools.empty(), "a pool group needs at least one pool");
  at::Tensor out = at::empty({(int64_t)(pools.size() * sizeof(barq_kv_pool))}, at::kByte);
  auto* dst = reinterpret_cast<barq_kv_pool*>(out.data_ptr<uint8_t>());
  const int64_t device = pools[0][0].get_device();
  for (size_t i = 0; i < pools.size(); ++i) {
    dst[i] = pool_from(pools[i]);
    TORCH_CHECK(pools[i][0].get_device() == device, "the pools of a group must share a device");
  }
  return out;
}

const barq_kv_pool* group_pools(const at::Tensor& group, int64_t* count) {
  TORCH_CHECK(group.device().is_cpu() && group.scalar_type() == at::kByte && group.is_contiguous() &&
                  group.numel() > 0 && group.numel() % (int64_t)sizeof(barq_kv_pool) == 0,
              "not a pool group (see pool_group)");
  *count = group.numel() / (int64_t)sizeof(barq_kv_pool);
  return reinterpret_cast<const barq_kv_pool*>(group.data_ptr<uint8_t>());
}

int64_t select_workspace_words(at::Tensor group, int64_t num_rows) {
  int64_t n = 0;
  const barq_kv_pool* pools = group_pools(group, &n);
  return barq_kv_select_workspace_words(pools, n, num_rows);
}

// rows: int32 on the pools' device; workspace: int32 of select_workspace_words(group, rows).
void pool_group_select_rows_(at::Tensor group, at::Tensor rows, at::Tensor workspace) {
  int64_t n = 0;
  const barq_kv_pool* pools = group_pools(group, &n);
  TORCH_CHECK(rows.is_cuda() && rows.scalar_type() == at::kInt && rows.is_contiguous(),
              "rows must be contiguous int32 on the pools' device");
  TORCH_CHECK(workspace.is_cuda() && workspace.scalar_type() == at::kInt && workspace.is_contiguous() &&
                  workspace.get_device() == rows.get_device(),
              "workspace must be contiguous int32 on the pools' device");
  c10::DeviceGuard guard(rows.device());
  check_status(barq_kv_select_rows_layers(pools, n, rows.data_ptr<int32_t>(), rows.numel(),
                                          workspace.data_ptr<int32_t>(), workspace.numel(), current_stream(rows)),
               "pool_group_select_rows_");
}

int64_t attention_workspace_bytes(std::vector<at::Tensor> pool, int64_t batch, int64_t q_heads,
                                  int64_t tokens, int64_t max_seq, int64_t split_tokens) {
  barq_kv_pool p = pool_from(pool);
  return barq_kv_attention_workspace_bytes(&p, batch, q_heads, tokens, max_seq, split_tokens);
}

// query [batch, q_heads, tokens, head_dim] in the pool's dtype; out of the same shape, in the
// pool's dtype or float32; workspace a zero-filled uint8 buffer (see
// barq_kv_decode_attention).
void decode_attention_into(const std::vector<at::Tensor>& pool, const barq_kv_cold* cold, const at::Tensor& query,
                           const at::Tensor& out, double scale, int64_t max_seq, int64_t split_tokens,
                           const at::Tensor& workspace) {
  barq_kv_pool p = pool_from(pool);
  const at::Tensor& pages = pool[0];
  TORCH_CHECK(pages.scalar_type() == at::kBFloat16 || pages.scalar_type() == at::kHalf,
              "paged decode attention needs a bfloat16 or float16 cache");
  TORCH_CHECK(query.is_cuda() && out.is_cuda() && workspace.is_cuda() &&
                  query.get_device() == pages.get_device() && out.get_device() == pages.get_device() &&
                  workspace.get_device() == pages.get_device(),
              "query, out and workspace must be on the cache device");
  TORCH_CHECK(query.dim() == 4 && query.scalar_type() == pages.scalar_type() && query.stride(3) == 1,
              "query must be [batch, q_heads, tokens, head_dim] in the cache dtype, head_dim contiguous");
  TORCH_CHECK(out.dim() == 4 && out.sizes() == query.sizes() && out.stride(3) == 1 &&
                  (out.scalar_type() == pages.scalar_type() || out.scalar_type() == at::kFloat),
              "out must match the query's shape, in the cache dtype or float32, head_dim contiguous");
  TORCH_CHECK(workspace.is_contiguous() && workspace.scalar_type() == at::kByte,
              "workspace must be a contiguous uint8 buffer");
  int64_t flags = 0;
  if (pages.scalar_type() == at::kHalf) flags |= BARQ_KV_ATTN_FP16;
  if (out.scalar_type() == at::kFloat) flags |= BARQ_KV_ATTN_OUT_F32;
  c10::DeviceGuard guard(pages.device());
  const int rc =
      cold ? barq_kv_decode_attention_cold(&p, cold, query.data_ptr(), query.size(0), query.size(1), query.size(2),
                                           query.stride(0), query.stride(1), query.stride(2), out.data_ptr(),
                                           out.stride(0), out.stride(1), out.stride(2), (float)scale, max_seq,
                                           split_tokens, flags, workspace.data_ptr(), workspace.numel(),
                                           current_stream(pages))
           : barq_kv_decode_attention(&p, query.data_ptr(), query.size(0), query.size(1), query.size(2),
                                      query.stride(0), query.stride(1), query.stride(2), out.data_ptr(),
                                      out.stride(0), out.stride(1), out.stride(2), (float)scale, max_seq,
                                      split_tokens, flags, workspace.data_ptr(), workspace.numel(),
                                      current_stream(pages));
  check_status(rc, "pool_decode_attention");
}

void pool_decode_attention(std::vector<at::Tensor> pool, at::Tensor query, at::Tensor out, double scale,
                           int64_t max_seq, int64_t split_tokens, at::Tensor workspace) {
  decode_attention_into(pool, nullptr, query, out, scale, max_seq, split_tokens, workspace);
}

// Decode attention over a pool with an fp8 cold store (quantised blocks read as codes).
void pool_decode_attention_cold(std::vector<at::Tensor> pool, std::vector<at::Tensor> cold, int64_t window,
                                at::Tensor query, at::Tensor out, double scale, int64_t max_seq,
                                int64_t split_tokens, at::Tensor workspace) {
  barq_kv_pool p = pool_from(pool);
  barq_kv_cold c = cold_from(p, pool[0], cold, window);
  decode_attention_into(pool, &c, query, out, scale, max_seq, split_tokens, workspace);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "BarqTrain paged KV cache on MI355X (gfx950): torch bindings of libbarq_kv.so";
  m.def("paged_kv_append_", &paged_kv_append_,
        "Append key/value states into the dense paged KV cache (HIP)");
  m.def("pool_reset_", &pool_reset_, "Empty a page pool", py::arg("pool"), py::arg("page_order") = py::none());
  m.def("pool_append_", &pool_append_, "Append tokens into a page pool");
  m.def("pool_gather", &pool_gather, "Materialise rows of a page pool as [B, H, S, D]");
  m.def("pool_update_", &pool_update_, "Append then materialise, in one pass");
  m.def("pool_crop_", &pool_crop_, "Clamp row lengths of a page pool");
  m.def("pool_free_rows_", &pool_free_rows_, "Return rows' pages to the free stack");
  m.def("pool_copy_rows_", &pool_copy_rows_, "Build rows of a fresh pool as copies of source rows");
  m.def("pool_select_rows_", &pool_select_rows_, "Rows become selected rows, sharing their full pages");
  m.def("pool_cold_reset_", &pool_cold_reset_, "Every page of a pool's fp8 cold store free");
  m.def("pool_compress_", &pool_compress_, "Quantise blocks behind the residual window into the cold store");
  m.def("pool_gather_cold", &pool_gather_cold, "Materialise rows of a pool with a cold store, dequantising");
  m.def("pool_update_cold_", &pool_update_cold_, "Append, compress, materialise (pool with a cold store)");
  m.def("pool_free_rows_cold_", &pool_free_rows_cold_, "Return rows' hot and cold pages");
  m.def("pool_crop_cold_", &pool_crop_cold_, "Clamp row lengths, re-opening quantised blocks past them");
  m.def("pool_select_rows_cold_", &pool_select_rows_cold_,
        "One row selection applied to pools with cold stores, sharing quantised blocks");
  m.def("pool_group", &pool_group, "Pack the pools of a model's layers for the batched entry points");
  m.def("pool_step_", &pool_step_, "One update / append with its host planning (see PagePool.update)");
  m.def("select_workspace_words", &select_workspace_words, "Workspace words of pool_group_select_rows_");
  m.def("pool_group_select_rows_", &pool_group_select_rows_,
        "One row selection applied to every pool of a group, sharing full pages");
  m.def("attention_workspace_bytes", &attention_workspace_bytes,
        "Workspace bytes of a decode-attention launch (-1: arguments rejected)");
  m.def("pool_decode_attention_cold", &pool_decode_attention_cold,
        "Decode attention reading a pool's quantised blocks as fp8 codes");
  m.def("pool_decode_attention", &pool_decode_attention,
        "Decode attention reading K/V from a page pool through its block table");
  m.def("version", []() { return std::string(barq_kv_version()); });
  m.attr("CTRL_WORDS") = BARQ_KV_CTRL_WORDS;
  m.attr("SEQ_FROM_DEVICE") = BARQ_KV_SEQ_FROM_DEVICE;
  m.attr("SEPARATE_FINALIZE") = BARQ_KV_SEPARATE_FINALIZE;
}
