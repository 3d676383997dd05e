// The sparse path's torch.library operators (namespace mdl_hip), in C++.
//
// This file is the PyTorch-ROCm extension of the package: it defines every
// mdl_hip schema and implements each operator for ROCm tensors by calling the
// C ABI of libmdl_hip.so (include/mdl_hip.h) on the current HIP stream.  The
// host work a training step repeats per table -- descriptor packing, the
// coalesced-gradient layout, the 200-odd sparse COO gradients of a backward,
// the optimizer's per-parameter checks, step counts and update records --
// runs here instead of in Python.  CPU kernels (the reference's CPU
// semantics) and fake kernels are registered by mdl_amd/library.py on these
// schemas; so is the autograd formula of the lookups.
//
// Replaces, on one GPU: the world==1 lookup loop of src/embeddings.py:1675-1709
// and its F.embedding calls (:438-473), the pooling of src/model.py:509-678,
// the sparse backward + coalesce of src/optim.py:321-324 and
// src/train.py:5730-5742, and ShardedRowWiseAdagrad.step (src/optim.py:299-377)
// with its fused update (:68-108).

#include <ATen/ATen.h>
#include <ATen/core/LegacyTypeDispatch.h>
#include <ATen/hip/EmptyTensor.h>
#include <ATen/SparseTensorImpl.h>
#include <ATen/native/SparseTensorUtils.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/core/DeviceGuard.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>
#include <c10/hip/HIPStream.h>
#include <c10/util/intrusive_ptr.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/csrc/autograd/function.h>
#include <torch/csrc/autograd/function_hook.h>
#include <torch/csrc/autograd/graph_task.h>
#include <torch/csrc/autograd/variable.h>
#include <torch/library.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <list>
#include <memory>
#include <mutex>
#include <numeric>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mdl_hip.h"

namespace mdl_torch {

using at::Tensor;
using at::TensorList;

// ---------------------------------------------------------------- basics --

constexpr int64_t kKeySpace = 0xFFFFFFFFll;  // sort keys are 32-bit; this one marks "no gradient"
constexpr int kForwardTargetIds = 480;       // ids per forward chunk at most (the LDS stage)

void check(int rc, const char* what) {
  if (rc != MDL_OK) {
    const char* msg = mdl_last_error();
    TORCH_CHECK(false, what, " failed (", rc, "): ", msg ? msg : "");
  }
}

void* stream_of(const at::Device& d) { return (void*)c10::hip::getCurrentHIPStream(d.index()).stream(); }

int dtype_code(at::ScalarType t) {
  if (t == at::kFloat) return MDL_F32;
  if (t == at::kBFloat16) return MDL_BF16;
  TORCH_CHECK_TYPE(false, "unsupported embedding dtype ", t, "; expected float32 or bfloat16");
  return -1;
}

uint64_t addr(const Tensor& t) { return (uint64_t)(uintptr_t)t.data_ptr(); }
template <typename T>
T* ptr_or_null(const std::optional<Tensor>& t) {
  return t.has_value() && t->defined() ? static_cast<T*>(t->data_ptr()) : nullptr;
}

void require_device(const Tensor& t, const char* what) {
  TORCH_CHECK(t.is_cuda(), what, " must live on a ROCm device; libmdl_hip has no host implementation");
}

// Host bytes -> device, through pinned memory, without a synchronisation (the
// caching host allocator keeps the staging block until the copy has run).
Tensor upload(const void* host, size_t bytes, const at::Device& dev) {
  const int64_t n = (int64_t)std::max<size_t>(bytes, 8);
  Tensor staged = at::empty({n}, at::TensorOptions().dtype(at::kByte).pinned_memory(true));
  if (bytes) std::memcpy(staged.data_ptr(), host, bytes);
  return staged.to(dev, at::kByte, /*non_blocking=*/true);
}

template <typename T>
Tensor upload_vec(const std::vector<T>& v, const at::Device& dev) {
  return upload(v.data(), v.size() * sizeof(T), dev);
}

Tensor workspace(size_t bytes, const at::Device& dev) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, at::TensorOptions().dtype(at::kByte).device(dev));
}

// A dense tensor over `base`'s storage (same device and key set) at a byte
// offset, built without a dispatcher call: the per-table rows and values of
// a backward are 200-odd such tensors per step.
Tensor raw_view(const Tensor& base, at::ScalarType dtype, int64_t byte_offset, at::IntArrayRef sizes,
                at::IntArrayRef strides) {
  const auto meta = c10::scalarTypeToTypeMeta(dtype);
  TORCH_CHECK(byte_offset % (int64_t)meta.itemsize() == 0, "view offset must be a multiple of the element size");
  auto impl = c10::make_intrusive<c10::TensorImpl>(c10::TensorImpl::VIEW, c10::Storage(base.storage()),
                                                   base.key_set(), meta);
  impl->set_sizes_and_strides(sizes, strides,
                              base.storage_offset() * (int64_t)base.element_size() / (int64_t)meta.itemsize() +
                                  byte_offset / (int64_t)meta.itemsize());
  return Tensor(std::move(impl));
}

int64_t bit_length(int64_t v) {
  int64_t b = 0;
  while (v > 0) {
    ++b;
    v >>= 1;
  }
  return b;
}

// ----------------------------------------------------------------- layouts --
//
// What a grouped call over the same tables (addresses, shapes, dtypes) and
// feature codes derives on the host, built once and kept in a small LRU:
// static feature descriptors, row bases, key groups and their table records.
// Entries hold addresses and sizes, never tensors, so a freed table keeps
// nothing alive.

struct KeyGroup {
  int lo = 0, hi = 0;          // features [lo, hi) of the (ordered) call
  std::vector<int> tables;     // global table indices, row bases counted from the group's first
  int64_t rows = 0;
  std::vector<mdl_table> recs; // the group's table records (feature indices local to the group)
  uint32_t classes = 0;
};

struct Layout {
  std::vector<mdl_feature> feats;  // static columns, call order (after `order`)
  std::vector<int64_t> row_base;   // per table, within its key group
  std::vector<KeyGroup> groups;
  std::vector<int> order;          // call feature f -> input feature order[f] (empty: identity)
  std::vector<int64_t> esz, dims;  // per table
  uint32_t sentinel = 0;
  int key_bits = 1;
  int max_dim = 1;
  bool pooled_any = false;
};

struct LayoutCache {
  std::mutex mu;
  using Key = std::vector<int64_t>;
  std::list<std::pair<Key, std::shared_ptr<const Layout>>> lru;  // most recent first
  std::unordered_multimap<uint64_t, decltype(lru)::iterator> index;
  static constexpr size_t kMax = 16;
};
LayoutCache g_layouts;

void validate_weights(TensorList weights) {
  TORCH_CHECK_VALUE(!weights.empty(), "a grouped lookup needs at least one table");
  const auto dev = weights[0].device();
  for (const Tensor& w : weights) {
    require_device(w, "embedding weight");
    TORCH_CHECK_VALUE(w.device() == dev, "every table of a grouped lookup lives on one device");
    TORCH_CHECK_VALUE(w.dim() == 2 && w.stride(1) == 1 && w.stride(0) == w.size(1),
                      "embedding weights must be contiguous [rows, dim] tensors");
    dtype_code(w.scalar_type());
    TORCH_CHECK_VALUE(w.size(0) < kKeySpace, "a table of a grouped lookup holds fewer than 2^32 - 1 rows");
  }
}

// Feature order of a device call: the caller's order (empty), except that a
// call over 2^32 - 1 table rows or more looks its features up sorted by
// table, so that each key group's features are consecutive (its keys one
// stretch).
std::vector<int> feature_order(int64_t total_rows, at::IntArrayRef table) {
  const int F = (int)table.size();
  if (total_rows < kKeySpace) return {};
  std::vector<int> ord(F);
  std::iota(ord.begin(), ord.end(), 0);
  std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return table[a] < table[b]; });
  bool identity = true;
  for (int f = 0; f < F; ++f) identity = identity && ord[f] == f;
  return identity ? std::vector<int>() : ord;
}

std::vector<int64_t> lookup_order(TensorList weights, at::IntArrayRef table) {
  int64_t total = 0;
  for (const Tensor& w : weights) total += w.size(0);
  auto ord = feature_order(total, table);
  return std::vector<int64_t>(ord.begin(), ord.end());
}

std::shared_ptr<const Layout> build_layout(TensorList weights, at::IntArrayRef table, at::IntArrayRef pooling,
                                           at::IntArrayRef exclude, at::IntArrayRef padding_idx) {
  const int T = (int)weights.size();
  const int F = (int)table.size();
  auto L = std::make_shared<Layout>();
  int64_t total = 0;
  for (const Tensor& w : weights) total += w.size(0);
  L->order = feature_order(total, table);
  auto src = [&](int f) { return L->order.empty() ? f : L->order[f]; };
  L->esz.resize(T);
  L->dims.resize(T);
  for (int t = 0; t < T; ++t) {
    L->esz[t] = weights[t].element_size();
    L->dims[t] = weights[t].size(1);
    L->max_dim = std::max<int>(L->max_dim, (int)weights[t].size(1));
  }
  // Key groups: one for a plan below 2^32 - 1 rows (row bases in table
  // order), else runs of consecutive features whose tables hold fewer rows
  // together (row bases counted from each group's first table).
  L->row_base.assign(T, 0);
  if (total < kKeySpace) {
    KeyGroup g;
    g.lo = 0;
    g.hi = F;
    int64_t base = 0;
    for (int t = 0; t < T; ++t) {
      g.tables.push_back(t);
      L->row_base[t] = base;
      base += weights[t].size(0);
    }
    g.rows = base;
    L->groups.push_back(std::move(g));
  } else {
    std::vector<int> owner(T, -1);
    KeyGroup cur;
    cur.lo = 0;
    for (int f = 0; f < F; ++f) {
      const int t = (int)table[src(f)];
      if (owner[t] >= 0) {
        TORCH_CHECK_VALUE(owner[t] == (int)L->groups.size(),
                          "a plan of 2^32 - 1 rows or more needs each table's features in one run of features "
                          "whose tables hold fewer rows than that (table ", t, " is read again by feature ", f, ")");
        continue;
      }
      const int64_t r = weights[t].size(0);
      if (!cur.tables.empty() && cur.rows + r >= kKeySpace) {
        cur.hi = f;
        L->groups.push_back(std::move(cur));
        cur = KeyGroup();
        cur.lo = f;
      }
      owner[t] = (int)L->groups.size();
      L->row_base[t] = cur.rows;
      cur.tables.push_back(t);
      cur.rows += r;
    }
    cur.hi = F;
    L->groups.push_back(std::move(cur));
  }
  int64_t sentinel = 0;
  for (const auto& g : L->groups) sentinel = std::max(sentinel, g.rows);
  L->sentinel = (uint32_t)sentinel;
  L->key_bits = (int)std::max<int64_t>(1, bit_length(sentinel));
  // Static feature columns.
  L->feats.assign(F, mdl_feature{});
  for (int f = 0; f < F; ++f) {
    const int i = src(f);
    const int t = (int)table[i];
    const Tensor& w = weights[t];
    mdl_feature& d = L->feats[f];
    d.weight = addr(w);
    d.num_rows = w.size(0);
    d.row_base = L->row_base[t];
    d.dim = (int32_t)w.size(1);
    d.wdtype = dtype_code(w.scalar_type());
    d.odtype = d.wdtype;
    d.pooling = (int32_t)pooling[i];
    d.flags = exclude[i] ? MDL_FLAG_EXCLUDE_NULL : 0;
    d.padding_idx = (int32_t)padding_idx[i];
    d.table = t;
    L->pooled_any = L->pooled_any || d.pooling != MDL_POOL_NONE;
  }
  // Table records of each group (a table read by one feature names it).
  for (auto& g : L->groups) {
    std::vector<int> local(T, -1);
    for (size_t j = 0; j < g.tables.size(); ++j) local[g.tables[j]] = (int)j;
    g.recs.assign(g.tables.size(), mdl_table{});
    std::vector<int> users(g.tables.size(), 0), user(g.tables.size(), -1);
    for (int f = g.lo; f < g.hi; ++f) {
      const int j = local[L->feats[f].table];
      users[j] += 1;
      user[j] = f - g.lo;
    }
    for (size_t j = 0; j < g.tables.size(); ++j) {
      const Tensor& w = weights[g.tables[j]];
      mdl_table& r = g.recs[j];
      r.weight = addr(w);
      r.state = 0;
      r.num_rows = w.size(0);
      r.row_base = L->row_base[g.tables[j]];
      r.dim = (int32_t)w.size(1);
      r.wdtype = dtype_code(w.scalar_type());
      r.feature = users[j] == 1 ? user[j] : -1;
      r.gdtype = r.wdtype;
    }
    g.classes = mdl_table_classes(g.recs.data(), (int32_t)g.recs.size());
  }
  return L;
}

uint64_t hash_key(const std::vector<int64_t>& k) {
  uint64_t h = 1469598103934665603ull;
  for (int64_t v : k) {
    h ^= (uint64_t)v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
    h *= 1099511628211ull;
  }
  return h;
}

// The cached layout of these tables and feature codes; the tables are
// validated when their layout is first built (the key holds everything the
// validation reads: address, shape, strides, dtype, device).
std::shared_ptr<const Layout> layout_for(TensorList weights, at::IntArrayRef table, at::IntArrayRef pooling,
                                         at::IntArrayRef exclude, at::IntArrayRef padding_idx) {
  LayoutCache::Key key;
  key.reserve(2 + weights.size() * 7 + 4 * (table.size() + 1));
  key.push_back((int64_t)weights.size());
  for (const Tensor& w : weights) {
    key.push_back((int64_t)addr(w));
    key.push_back(w.dim());
    key.push_back(w.dim() == 2 ? w.size(0) : -1);
    key.push_back(w.dim() == 2 ? w.size(1) : -1);
    key.push_back(w.dim() == 2 ? w.stride(0) : -1);
    key.push_back(w.dim() == 2 ? w.stride(1) : -1);
    key.push_back(((int64_t)w.scalar_type() << 16) | ((int64_t)w.device().type() << 8) | (w.device().index() & 0xff));
  }
  for (auto arr : {table, pooling, exclude, padding_idx}) {
    key.push_back(-7);
    key.insert(key.end(), arr.begin(), arr.end());
  }
  const uint64_t h = hash_key(key);
  {
    std::lock_guard<std::mutex> lock(g_layouts.mu);
    auto range = g_layouts.index.equal_range(h);
    for (auto it = range.first; it != range.second; ++it) {
      if (it->second->first == key) {
        g_layouts.lru.splice(g_layouts.lru.begin(), g_layouts.lru, it->second);
        return it->second->second;
      }
    }
  }
  validate_weights(weights);
  auto L = build_layout(weights, table, pooling, exclude, padding_idx);
  std::lock_guard<std::mutex> lock(g_layouts.mu);
  g_layouts.lru.emplace_front(std::move(key), L);
  g_layouts.index.emplace(h, g_layouts.lru.begin());
  if (g_layouts.lru.size() > LayoutCache::kMax) {
    const uint64_t old = hash_key(g_layouts.lru.back().first);
    auto range = g_layouts.index.equal_range(old);
    for (auto it = range.first; it != range.second; ++it) {
      if (it->second == std::prev(g_layouts.lru.end())) {
        g_layouts.index.erase(it);
        break;
      }
    }
    g_layouts.lru.pop_back();
  }
  return L;
}

void check_features(TensorList weights, TensorList ids, const c10::List<std::optional<Tensor>>& lengths,
                    at::IntArrayRef table, at::IntArrayRef pooling, at::IntArrayRef exclude,
                    at::IntArrayRef padding_idx) {
  const size_t nf = ids.size();
  TORCH_CHECK_VALUE(lengths.size() == nf && table.size() == nf && pooling.size() == nf && exclude.size() == nf &&
                        padding_idx.size() == nf,
                    "one entry per feature in ids, lengths, table, pooling, exclude and padding_idx");
  for (size_t f = 0; f < nf; ++f) {
    TORCH_CHECK_TYPE(ids[f].scalar_type() == at::kLong, "sharded embedding indices must be torch.long");
    TORCH_CHECK_VALUE(table[f] >= 0 && table[f] < (int64_t)weights.size(), "feature table index out of range");
    TORCH_CHECK_VALUE(pooling[f] >= 0 && pooling[f] <= 2, "unsupported pooling code ", pooling[f]);
    if (pooling[f] != 0) {
      const std::optional<Tensor> ln = lengths.get(f);
      TORCH_CHECK_VALUE(ln.has_value() && ln->defined() && ln->dim() == 1,
                        "categorical bag lengths must have shape [B]");
    }
  }
}

int forward_target_ids(int64_t n) {
  return (int)std::max<int64_t>(96, std::min<int64_t>(kForwardTargetIds, n / 3072));
}

// Per-call descriptor columns (build_features): output/gradient rows, id and
// bag placement.  rows_out[f] is the output rows of feature f.
std::vector<mdl_feature> call_features(const Layout& L, const std::vector<int64_t>& n_ids,
                                       const std::vector<int64_t>& n_bags, std::vector<int64_t>* rows_out) {
  const int F = (int)L.feats.size();
  std::vector<mdl_feature> feats = L.feats;
  int64_t payload = 0, ids_begin = 0, bag_base = 0;
  if (rows_out) rows_out->assign(F, 0);
  for (int f = 0; f < F; ++f) {
    mdl_feature& d = feats[f];
    const bool pooled = d.pooling != MDL_POOL_NONE;
    const int64_t rows = pooled ? n_bags[f] : n_ids[f];
    d.payload_base = payload;
    d.ids_begin = ids_begin;
    d.bag_base = bag_base;
    d.num_ids = n_ids[f];
    d.num_bags = pooled ? n_bags[f] : 0;
    payload += rows;
    ids_begin += n_ids[f];
    bag_base += pooled ? n_bags[f] : (L.pooled_any ? 1 : 0);
    if (rows_out) (*rows_out)[f] = rows;
  }
  TORCH_CHECK_VALUE(payload < kKeySpace, "a grouped lookup supports fewer than 2^32 - 1 output rows");
  return feats;
}

template <typename T>
std::vector<T> permute(const std::vector<T>& v, const std::vector<int>& order) {
  if (order.empty()) return v;
  std::vector<T> out(order.size());
  for (size_t f = 0; f < order.size(); ++f) out[f] = v[order[f]];
  return out;
}

// ------------------------------------------------------------ grouped lookup --

std::tuple<std::vector<Tensor>, Tensor, Tensor, Tensor, Tensor, Tensor> grouped_lookup_cuda(
    TensorList weights, TensorList ids_in, const c10::List<std::optional<Tensor>>& lengths_in,
    at::IntArrayRef table, at::IntArrayRef pooling, at::IntArrayRef exclude, at::IntArrayRef padding_idx,
    bool need_backward) {
  TORCH_CHECK_VALUE(!weights.empty(), "a grouped lookup needs at least one table");
  check_features(weights, ids_in, lengths_in, table, pooling, exclude, padding_idx);
  const at::Device dev = weights[0].device();
  const c10::DeviceGuard guard(dev);
  auto L = layout_for(weights, table, pooling, exclude, padding_idx);
  const int F = (int)ids_in.size();
  std::vector<Tensor> ids(F);
  std::vector<std::optional<Tensor>> lengths(F);
  for (int f = 0; f < F; ++f) {
    const int i = L->order.empty() ? f : L->order[f];
    ids[f] = ids_in[i];
    require_device(ids[f], "ids");
    lengths[f] = lengths_in.get(i);
  }
  std::vector<int64_t> n_ids(F), n_bags(F, 0);
  int64_t n = 0;
  for (int f = 0; f < F; ++f) {
    n_ids[f] = ids[f].numel();
    n += n_ids[f];
    if (L->feats[f].pooling != MDL_POOL_NONE) n_bags[f] = lengths[f]->numel();
  }
  void* s = stream_of(dev);
  // Every feature's ids back to back; the offsets of all features from one
  // scan of the concatenated lengths (an unpooled feature's pseudo-length is
  // its id count).
  // Id tensors that lie back to back in one buffer (a packed loader batch)
  // are used where they are; others are concatenated.
  bool packed = true;
  for (int f = 0; f < F && packed; ++f) {
    const Tensor& t = ids[f];
    packed = t.is_contiguous() && t.scalar_type() == at::kLong &&
             (f == 0 || (t.numel() == 0 && n_ids[f] == 0) ||
              (ids[f - 1].storage().is_alias_of(t.storage()) &&
               addr(t) == addr(ids[f - 1]) + 8 * (uint64_t)n_ids[f - 1]));
  }
  Tensor all_ids;
  if (packed) {
    all_ids = raw_view(ids[0], at::kLong, 0, {n}, {1});
  } else {
    std::vector<Tensor> flat;
    flat.reserve(F);
    for (const Tensor& t : ids)
      flat.push_back(t.is_contiguous() ? raw_view(t, at::kLong, 0, {t.numel()}, {1}) : t.reshape({-1}));
    all_ids = F == 1 ? flat[0].contiguous() : at::cat(flat).contiguous();
  }
  Tensor ids_arg = n ? all_ids : at::zeros({1}, all_ids.options());
  Tensor offsets;
  if (L->pooled_any) {
    std::vector<int64_t> pseudo;
    for (int f = 0; f < F; ++f)
      if (L->feats[f].pooling == MDL_POOL_NONE) pseudo.push_back(n_ids[f]);
    Tensor pseudo_dev;
    if (!pseudo.empty()) pseudo_dev = upload_vec(pseudo, dev).view(at::kLong).narrow(0, 0, (int64_t)pseudo.size());
    std::vector<Tensor> parts;
    parts.reserve(F);
    int64_t k = 0;
    for (int f = 0; f < F; ++f) {
      if (L->feats[f].pooling != MDL_POOL_NONE) {
        const Tensor& ln = *lengths[f];
        require_device(ln, "bag lengths");
        parts.push_back(ln.scalar_type() == at::kLong ? ln : ln.to(at::kLong));
      } else {
        parts.push_back(pseudo_dev.narrow(0, k++, 1));
      }
    }
    Tensor len_all = (F == 1 ? parts[0] : at::cat(parts)).contiguous();
    const int64_t nl = len_all.numel();
    offsets = at::empty({nl + 1}, len_all.options());
    Tensor ws = workspace(mdl_offsets_workspace_bytes(nl), dev);
    check(mdl_lengths_to_offsets(len_all.data_ptr<int64_t>(), nl, offsets.data_ptr<int64_t>(), ws.data_ptr(),
                                 (size_t)ws.numel(), s),
          "mdl_lengths_to_offsets");
  }
  std::vector<int64_t> rows_out;
  std::vector<mdl_feature> feats = call_features(*L, n_ids, n_bags, &rows_out);
  // One tensor per output (a functional op's outputs may not share storage).
  std::vector<Tensor> outputs(F);
  int64_t total_rows = 0;
  for (int f = 0; f < F; ++f) {
    const Tensor& w = weights[L->feats[f].table];
    const int64_t dim = w.size(1);
    std::vector<int64_t> shape;
    if (L->feats[f].pooling == MDL_POOL_NONE) {
      shape = ids[f].sizes().vec();
      shape.push_back(dim);
    } else {
      shape = {n_bags[f], dim};
    }
    // every element is written by the lookup: allocated without a dispatcher
    // round trip per output
    outputs[f] = w.is_cuda() ? Tensor(at::detail::empty_cuda(shape, w.scalar_type(), dev, std::nullopt))
                             : at::empty(shape, w.options());
    feats[f].out = addr(outputs[f]);
    feats[f].out_stride = dim;
    total_rows += rows_out[f];
  }
  const int target = forward_target_ids(n);
  const int64_t n_chunks = mdl_plan_chunks(feats.data(), F, target, nullptr, 0);
  if (n_chunks < 0) check((int)n_chunks, "mdl_plan_chunks");
  // one upload: descriptors, then chunks (16-byte records after 128-byte ones)
  const size_t fbytes = feats.size() * sizeof(mdl_feature);
  std::vector<uint8_t> host(fbytes + std::max<int64_t>(n_chunks, 1) * sizeof(mdl_chunk));
  std::memcpy(host.data(), feats.data(), fbytes);
  mdl_chunk* chunks = reinterpret_cast<mdl_chunk*>(host.data() + fbytes);
  if (n_chunks > 0) mdl_plan_chunks(feats.data(), F, target, chunks, n_chunks);
  Tensor meta = upload(host.data(), host.size(), dev);
  const uint32_t classes = mdl_feature_classes(feats.data(), F);
  auto i32 = at::TensorOptions().dtype(at::kInt).device(dev);
  Tensor err = at::zeros({1}, i32);
  Tensor keys = at::empty({0}, i32), payload = at::empty({0}, i32);
  if (need_backward) {
    keys = n ? at::empty({n}, i32) : at::zeros({1}, i32);
    payload = n ? at::empty({n}, i32) : at::zeros({1}, i32);
  }
  Tensor bag_count = at::empty({0}, at::TensorOptions().dtype(at::kFloat).device(dev));
  if (L->pooled_any) bag_count = at::zeros({std::max<int64_t>(total_rows, 1)}, bag_count.options());
  uint8_t* mbase = static_cast<uint8_t*>(meta.data_ptr());
  check(mdl_forward(reinterpret_cast<const mdl_feature*>(mbase), F, reinterpret_cast<const mdl_chunk*>(mbase + fbytes),
                    n_chunks, ids_arg.data_ptr<int64_t>(), n, offsets.defined() ? offsets.data_ptr<int64_t>() : nullptr,
                    need_backward ? reinterpret_cast<uint32_t*>(keys.data_ptr()) : nullptr,
                    need_backward ? reinterpret_cast<uint32_t*>(payload.data_ptr()) : nullptr, nullptr, L->sentinel,
                    L->pooled_any ? bag_count.data_ptr<float>() : nullptr, err.data_ptr<int32_t>(), classes, s),
        "mdl_forward");
  if (!offsets.defined()) offsets = at::empty({0}, at::TensorOptions().dtype(at::kLong).device(dev));
  if (!L->order.empty()) {
    std::vector<Tensor> back(F);
    for (int f = 0; f < F; ++f) back[L->order[f]] = outputs[f];
    outputs = std::move(back);
  }
  return {outputs, keys, payload, bag_count, offsets, err};
}

// The modules' forward: mdl_hip::grouped_lookup called below the autograd
// keys, for callers that record the autograd graph themselves (the modules
// keep one node per call over the tables).  Through the op's own autograd
// registration, a Python wrapper that flattens every list argument, a call
// of 150 features cost about 0.2 ms more.
std::tuple<std::vector<Tensor>, Tensor, Tensor, Tensor, Tensor, Tensor> grouped_lookup_untracked(
    TensorList weights, TensorList ids, const c10::List<std::optional<Tensor>>& lengths, at::IntArrayRef table,
    at::IntArrayRef pooling, at::IntArrayRef exclude, at::IntArrayRef padding_idx, bool need_backward) {
  static auto op = c10::Dispatcher::singleton()
                       .findSchemaOrThrow("mdl_hip::grouped_lookup", "")
                       .typed<std::tuple<std::vector<Tensor>, Tensor, Tensor, Tensor, Tensor, Tensor>(
                           TensorList, TensorList, const c10::List<std::optional<Tensor>>&, at::IntArrayRef,
                           at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, bool)>();
  at::AutoDispatchBelowAutograd below;
  return op.call(weights, ids, lengths, table, pooling, exclude, padding_idx, need_backward);
}

// --------------------------------------------------- coalesced gradients --
//
// Capacity-sized coalesced gradients of every table in two flat buffers:
// table t's rows at rows_off[t] (int64 elements), its values at byte
// val_off[t] (each table's region 256-byte aligned).  cap[t] bounds its
// distinct rows (its id count, known from the shapes).

struct CoalescedLayout {
  std::vector<int64_t> cap, nbytes, rows_off, val_off;
};

CoalescedLayout coalesced_layout(const std::vector<int64_t>& esz, const std::vector<int64_t>& dims,
                                 const std::vector<int64_t>& cap) {
  const size_t T = cap.size();
  CoalescedLayout c;
  c.cap = cap;
  c.nbytes.resize(T);
  c.rows_off.assign(T + 1, 0);
  c.val_off.assign(T + 1, 0);
  for (size_t t = 0; t < T; ++t) {
    c.nbytes[t] = cap[t] * dims[t] * esz[t];
    c.rows_off[t + 1] = c.rows_off[t] + cap[t];
    c.val_off[t + 1] = c.val_off[t] + (c.nbytes[t] + 255) / 256 * 256;
  }
  return c;
}

// Gradient rows of feature f as the kernels read them: the feature's dtype,
// 2-D, unit column stride, 16-byte aligned rows where the row size allows.
Tensor attach_grad(const Tensor& g_in, const Layout& L, int f, const std::vector<int64_t>& rows_out) {
  const mdl_feature& d = L.feats[f];
  const auto out_dtype = d.odtype == MDL_F32 ? at::kFloat : at::kBFloat16;
  TORCH_CHECK_VALUE(g_in.defined() && g_in.numel() == rows_out[f] * d.dim,
                    "the gradient of feature ", f, " must hold its output's ", rows_out[f], " rows of ", d.dim);
  Tensor g = g_in;
  require_device(g, "gradient");
  if (g.scalar_type() != out_dtype) g = g.to(out_dtype);
  Tensor g2 = g.dim() == 2 ? g : g.reshape({-1, (int64_t)d.dim});
  const int64_t es = g2.element_size();
  if ((d.dim * es) % 16 == 0 &&
      (g2.stride(-1) != 1 || addr(g2) % 16 != 0 || (g2.stride(0) * es) % 16 != 0)) {
    g2 = g2.contiguous();
    if (addr(g2) % 16 != 0) g2 = g2.clone();
  }
  if (g2.stride(-1) != 1) g2 = g2.contiguous();
  return g2;
}

// The backward's key groups: descriptors, tables and their stretch of keys.
struct CoalesceResult {
  Tensor rows_all, vbuf, counts;
  CoalescedLayout layout;
};

// Sort, count and coalesce every key group of a call.  The counting kernels
// of all groups go first (each group keeps its own workspace, which its
// coalescing reduce reads), so a caller that needs the row counts on the host
// (`host_counts`) reads them before the reduces are queued: it waits for the
// sort and the count only, and builds its tensors while the reduces run.
// `pad` fills entries [U_t, cap_t) of every table (capacity-sized
// gradients); exact gradients do not view them.
CoalesceResult coalesce_groups(const Layout& L, std::vector<mdl_feature>& feats, const Tensor& keys,
                               const Tensor& payload, const Tensor& bag_count, const std::vector<int64_t>& cap,
                               const at::Device& dev, bool pad = true, std::vector<int64_t>* host_counts = nullptr) {
  void* s = stream_of(dev);
  const int T = (int)L.esz.size();
  CoalesceResult r;
  r.layout = coalesced_layout(L.esz, L.dims, cap);
  const auto& lay = r.layout;
  r.rows_all = at::empty({std::max<int64_t>(lay.rows_off[T], 1)}, at::TensorOptions().dtype(at::kLong).device(dev));
  r.vbuf = at::empty({std::max<int64_t>(lay.val_off[T], 1)}, at::TensorOptions().dtype(at::kByte).device(dev));
  int64_t n_ranges = 0;
  for (const auto& g : L.groups) n_ranges += 2 * (int64_t)g.tables.size();
  Tensor urange = at::zeros({n_ranges}, at::TensorOptions().dtype(at::kLong).device(dev));
  const uint64_t rows_base = addr(r.rows_all), vals_base = addr(r.vbuf);
  struct Launch {
    const mdl_feature* fd;
    const mdl_table* td;
    const int64_t* md;
    int Tg, nf;
    int64_t n, units;
    int64_t* ur;
    uint32_t *k, *p;
    Tensor dmeta, ws;
    uint32_t classes;
  };
  std::vector<Launch> launches;
  int64_t u0 = 0;
  for (const auto& g : L.groups) {
    const int Tg = (int)g.tables.size();
    int64_t* ur = urange.data_ptr<int64_t>() + u0;
    u0 += 2 * Tg;
    int64_t n = 0;
    for (int f = g.lo; f < g.hi; ++f) n += feats[f].num_ids;
    if (!n) continue;
    const int64_t first = feats[g.lo].ids_begin;
    // one upload: row and value addresses, capacities, pad-unit prefix
    std::vector<int64_t> meta(4 * Tg + 1, 0);
    for (int j = 0; j < Tg; ++j) {
      const int t = g.tables[j];
      const int64_t c = cap[t];
      meta[j] = c > 0 ? (int64_t)(rows_base + 8 * lay.rows_off[t]) : 0;
      meta[Tg + j] = c > 0 ? (int64_t)(vals_base + lay.val_off[t]) : 0;
      meta[2 * Tg + j] = c;
      meta[3 * Tg + j + 1] = meta[3 * Tg + j] + (c + 63) / 64;
    }
    const size_t fbytes = (size_t)(g.hi - g.lo) * sizeof(mdl_feature);
    const size_t tbytes = (size_t)Tg * sizeof(mdl_table);
    const size_t mbytes = meta.size() * 8;
    std::vector<uint8_t> host(fbytes + tbytes + mbytes);
    std::memcpy(host.data(), feats.data() + g.lo, fbytes);
    std::memcpy(host.data() + fbytes, g.recs.data(), tbytes);
    std::memcpy(host.data() + fbytes + tbytes, meta.data(), mbytes);
    Launch l;
    l.dmeta = upload(host.data(), host.size(), dev);
    const uint8_t* b = static_cast<const uint8_t*>(l.dmeta.data_ptr());
    l.fd = reinterpret_cast<const mdl_feature*>(b);
    l.td = reinterpret_cast<const mdl_table*>(b + fbytes);
    l.md = reinterpret_cast<const int64_t*>(b + fbytes + tbytes);
    l.Tg = Tg;
    l.nf = g.hi - g.lo;
    l.n = n;
    l.units = meta[4 * Tg];
    l.ur = ur;
    l.k = reinterpret_cast<uint32_t*>(keys.data_ptr()) + first;
    l.p = reinterpret_cast<uint32_t*>(payload.data_ptr()) + first;
    l.ws = workspace(mdl_backward_workspace_bytes(n, Tg, L.max_dim), dev);
    l.classes = g.classes;
    check(mdl_backward_count(l.td, Tg, L.max_dim, l.k, l.p, n, nullptr, L.key_bits, ur, l.ws.data_ptr(),
                             (size_t)l.ws.numel(), s),
          "mdl_backward_count");
    launches.push_back(std::move(l));
  }
  Tensor diff = urange.slice(0, 1, n_ranges, 2) - urange.slice(0, 0, n_ranges, 2);
  if (L.groups.size() == 1) {
    r.counts = diff;
  } else {
    std::vector<int64_t> order;
    for (const auto& g : L.groups)
      for (int t : g.tables) order.push_back(t);
    r.counts = at::zeros({T}, urange.options());
    r.counts.index_copy_(0, upload_vec(order, dev).view(at::kLong).narrow(0, 0, (int64_t)order.size()), diff);
  }
  if (host_counts) {
    Tensor h = r.counts.to(at::kCPU);
    host_counts->assign(h.data_ptr<int64_t>(), h.data_ptr<int64_t>() + T);
  }
  for (const Launch& l : launches) {
    check(mdl_backward_coalesce(l.fd, l.nf, l.td, l.Tg, L.max_dim, l.k, l.p, l.n, L.key_bits,
                                bag_count.defined() && bag_count.numel() ? bag_count.data_ptr<float>() : nullptr, l.ur,
                                reinterpret_cast<const uint64_t*>(l.md), reinterpret_cast<const uint64_t*>(l.md + l.Tg),
                                l.ws.data_ptr(), (size_t)l.ws.numel(), l.classes, s),
          "mdl_backward_coalesce");
    if (pad)
      check(mdl_backward_pad(l.td, l.Tg, l.ur, reinterpret_cast<const uint64_t*>(l.md),
                             reinterpret_cast<const uint64_t*>(l.md + l.Tg), l.md + 2 * l.Tg, l.md + 3 * l.Tg, l.units,
                             s),
            "mdl_backward_pad");
  }
  return r;
}

// The grouped lookup's backward on the device.  `sort_in_place` sorts the
// forward's keys and payloads where they are (the modules' own backward: a
// second backward over a retained graph sorts the sorted pairs again, to the
// same order); the public op sorts copies and leaves its inputs as they are.
CoalesceResult lookup_backward(TensorList weights, TensorList ids_in,
                               const c10::List<std::optional<Tensor>>& lengths_in, at::IntArrayRef table,
                               at::IntArrayRef pooling, at::IntArrayRef exclude, at::IntArrayRef padding_idx,
                               TensorList grads_in, const Tensor& keys_in, const Tensor& payload_in,
                               const Tensor& bag_count, bool sort_in_place, bool pad,
                               std::vector<int64_t>* host_counts) {
  TORCH_CHECK_VALUE(!weights.empty(), "a grouped lookup needs at least one table");
  check_features(weights, ids_in, lengths_in, table, pooling, exclude, padding_idx);
  TORCH_CHECK_VALUE(grads_in.size() == ids_in.size(), "one gradient per feature");
  const at::Device dev = weights[0].device();
  const c10::DeviceGuard guard(dev);
  auto L = layout_for(weights, table, pooling, exclude, padding_idx);
  const int F = (int)ids_in.size();
  const int T = (int)weights.size();
  std::vector<int64_t> n_ids(F), n_bags(F, 0), cap(T, 0);
  int64_t n = 0;
  for (int f = 0; f < F; ++f) {
    const int i = L->order.empty() ? f : L->order[f];
    n_ids[f] = ids_in[i].numel();
    n += n_ids[f];
    if (L->feats[f].pooling != MDL_POOL_NONE) n_bags[f] = lengths_in.get(i)->numel();
    cap[L->feats[f].table] += n_ids[f];
  }
  TORCH_CHECK_VALUE(keys_in.numel() >= n && payload_in.numel() >= n,
                    "sort keys and payloads hold one entry per looked-up id");
  Tensor keys = sort_in_place ? keys_in : keys_in.clone();
  Tensor payload = sort_in_place ? payload_in : payload_in.clone();
  std::vector<int64_t> rows_out;
  std::vector<mdl_feature> feats = call_features(*L, n_ids, n_bags, &rows_out);
  std::vector<Tensor> grads(F);
  for (int f = 0; f < F; ++f) {
    const int i = L->order.empty() ? f : L->order[f];
    grads[f] = attach_grad(grads_in[i], *L, f, rows_out);
    feats[f].grad = addr(grads[f]);
    feats[f].out = addr(grads[f]);
    feats[f].out_stride = grads[f].stride(0);
  }
  return coalesce_groups(*L, feats, keys, payload, bag_count, cap, dev, pad, host_counts);
}

std::tuple<Tensor, Tensor, Tensor> grouped_lookup_backward_cuda(
    TensorList weights, TensorList ids_in, const c10::List<std::optional<Tensor>>& lengths_in,
    at::IntArrayRef table, at::IntArrayRef pooling, at::IntArrayRef exclude, at::IntArrayRef padding_idx,
    TensorList grads_in, const Tensor& keys_in, const Tensor& payload_in, const Tensor& bag_count,
    const Tensor& offsets) {
  CoalesceResult r = lookup_backward(weights, ids_in, lengths_in, table, pooling, exclude, padding_idx, grads_in,
                                     keys_in, payload_in, bag_count, false, true, nullptr);
  return {r.rows_all, r.vbuf, r.counts};
}

}  // namespace mdl_torch

namespace mdl_torch {

// --------------------------------------------------- gradients as records --
//
// A capacity-sized gradient (table t: cap_t entries, the first U_t coalesced,
// the rest the last row again with zero values) is a valid uncoalesced COO
// tensor of the right sum whose size needs no host read.  The optimizer still
// has to update exactly the U_t live rows, so the backward records
// (rows, values, device count) under the parameter; the step matches the
// record to the parameter's gradient by storage (autograd's AccumulateGrad
// re-wraps the same index and value storage) and reads the count on the
// device.  A gradient that matches no record (accumulated over several
// backward passes, or built elsewhere) is coalesced again.

struct CapRecord {
  c10::weak_intrusive_ptr<c10::TensorImpl> param;
  Tensor rows, values, count;
};
std::mutex g_cap_mu;
std::unordered_map<const c10::TensorImpl*, CapRecord> g_cap;

void drop_dead_records();

void note_capacity_grad(const Tensor& param, const Tensor& rows, const Tensor& values, const Tensor& count) {
  g_cap.insert_or_assign(param.unsafeGetTensorImpl(),
                         CapRecord{c10::weak_intrusive_ptr<c10::TensorImpl>(param.getIntrusivePtr()), rows, values,
                                   count});
}

// (rows, values, count) when grad is the capacity-sized gradient last
// recorded for param.
std::optional<std::tuple<Tensor, Tensor, Tensor>> find_capacity_grad(const Tensor& param, const Tensor& grad) {
  auto it = g_cap.find(param.unsafeGetTensorImpl());
  if (it == g_cap.end() || it->second.param.expired()) return std::nullopt;
  const CapRecord& r = it->second;
  if (!grad.is_sparse()) return std::nullopt;
  const auto* sp = at::sparse::get_sparse_impl(grad);
  const Tensor& idx = sp->indices();
  const Tensor& val = sp->values();
  if (idx.data_ptr() == r.rows.data_ptr() && val.data_ptr() == r.values.data_ptr() && idx.size(-1) == r.rows.numel() &&
      val.sizes() == r.values.sizes())
    return std::make_tuple(r.rows, r.values, r.count);
  return std::nullopt;
}

// Exact coalesced gradients keep their flag on the parameter.  Autograd's
// AccumulateGrad re-wraps a first sparse gradient around the same index and
// value storage without its coalesced flag (torch's accumulate_grad.h, "Case
// 1.2"), which would make the trainer's grad.coalesce() sort it again.  A
// post-accumulate hook, installed once on a parameter that has none, marks
// the parameter's gradient coalesced when it is the tensor just emitted
// (same value storage and entry count); a gradient summed over several
// backward passes is not that tensor and is left as it is.
struct ExactRecord {
  c10::weak_intrusive_ptr<c10::TensorImpl> param;
  const void* values;
  int64_t nnz;
};
std::unordered_map<const c10::TensorImpl*, ExactRecord> g_exact;

struct MarkCoalesced final : torch::autograd::PostAccumulateGradHook {
  void operator()(const torch::autograd::Variable& p) override {
    const Tensor& g = p.grad();
    std::lock_guard<std::mutex> lock(g_cap_mu);
    auto it = g_exact.find(p.unsafeGetTensorImpl());
    if (it == g_exact.end()) return;
    const ExactRecord r = it->second;
    g_exact.erase(it);
    if (!g.defined() || !g.is_sparse()) return;
    auto* sp = at::sparse::get_sparse_impl(g);
    if (sp->nnz() == r.nnz && (r.nnz == 0 || sp->values().data_ptr() == r.values)) sp->set_coalesced(true);
  }
};

void drop_dead_records() {
  for (auto it = g_cap.begin(); it != g_cap.end();) {
    if (it->second.param.expired()) it = g_cap.erase(it);
    else ++it;
  }
  for (auto it = g_exact.begin(); it != g_exact.end();) {
    if (it->second.param.expired()) it = g_exact.erase(it);
    else ++it;
  }
}

// Under g_cap_mu.
void note_exact_grad(const Tensor& param, const Tensor& values) {
  if (!param.requires_grad()) return;
  g_exact.insert_or_assign(param.unsafeGetTensorImpl(),
                           ExactRecord{c10::weak_intrusive_ptr<c10::TensorImpl>(param.getIntrusivePtr()),
                                       values.data_ptr(), values.size(0)});
  auto& hook = torch::autograd::impl::post_acc_grad_hooks(param);
  if (!hook) torch::autograd::impl::set_post_acc_grad_hooks(param, std::make_unique<MarkCoalesced>());
}

// A [num_rows, dim] sparse COO tensor (sparse_dim 1, dense_dim 1) over
// `rows` (as a [1, n] index view) and `values`, built as ATen's own
// constructors build one but without their dispatcher round trips.
Tensor sparse_grad(const Tensor& weight, const Tensor& rows, const Tensor& values, bool coalesced) {
  const auto key = values.is_cuda() ? c10::DispatchKey::SparseCUDA : c10::DispatchKey::SparseCPU;
  Tensor t = at::detail::make_tensor<at::SparseTensorImpl>(c10::DispatchKeySet(key), values.dtype());
  auto* impl = at::sparse::get_sparse_impl(t);
  // sizes and dims only: the indices and values set next fit them
  impl->raw_resize_(1, 1, weight.sizes());
  const int64_t n = rows.numel();
  impl->set_indices_and_values_unsafe(raw_view(rows, at::kLong, 0, {1, n}, {n, 1}), values);
  impl->set_coalesced(coalesced);
  return t;
}

// Autograd's AccumulateGrad stores a parameter's first sparse gradient as a
// new COO tensor around the same indices and values (torch's
// accumulate_grad.h, "Case 1.2"): a dispatcher call and a tensor per table,
// the largest host cost left in a training step over hundreds of tables.
// The backward stores such a first gradient on the parameter itself, and
// hands autograd none for it, only where nothing can tell the two apart:
// grad mode off (no create_graph) in a backward() that runs every
// accumulator (not autograd.grad or backward(inputs=...), which select or
// capture gradients), a leaf that has no gradient yet, no hook of any kind
// on the leaf or its accumulator (the library's own post-accumulate hook
// aside), and an accumulator that runs on the current stream, so the
// gradient is ready where AccumulateGrad would have put it.  Anything else
// takes autograd's path.
bool plain_backward() {
  if (at::GradMode::is_enabled()) return false;
  const auto* info = torch::autograd::get_current_graph_task_exec_info();
  return info != nullptr && info->empty();
}

bool stores_first_grad(const Tensor& w) {
  if (!w.is_leaf() || !w.requires_grad() || w.grad().defined()) return false;
  std::shared_ptr<torch::autograd::Node> acc = torch::autograd::impl::try_get_grad_accumulator(w);
  if (!acc || !acc->pre_hooks().empty() || !acc->post_hooks().empty() || !acc->tensor_pre_hooks().empty() ||
      !acc->retains_grad_hooks().empty())
    return false;
  const auto& post = torch::autograd::impl::post_acc_grad_hooks(w);
  if (post && !dynamic_cast<const MarkCoalesced*>(post.get())) return false;
  // the current stream as autograd records streams (a ROCm stream under the
  // CUDA device type, which HIPStream::unwrap does not give)
  std::optional<c10::Stream> current;
  if (!w.is_cpu()) current = c10::impl::getDeviceGuardImpl(w.device().type())->getStream(w.device());
  return acc->stream() == current;
}

// Per-table gradients from the two flat buffers: capacity-sized and recorded
// (no host read), or -- `coalesced` -- cut to their row counts after one
// batched read of the counts and marked coalesced, so coalesce() returns them
// as they are (src/optim.py:321-324, src/train.py:5730-5742).  A gradient
// stored on its parameter (stores_first_grad) comes back undefined.
std::vector<std::optional<Tensor>> weight_grads(TensorList weights, const Tensor& rows_all, const Tensor& vbuf,
                                                const Tensor& counts, const CoalescedLayout& lay, bool coalesced,
                                                const std::vector<int64_t>* host_counts = nullptr) {
  const int T = (int)weights.size();
  std::vector<std::optional<Tensor>> out(T);
  std::vector<int64_t> u(T, 0);
  if (coalesced && host_counts) {
    u = *host_counts;
  } else if (coalesced) {
    Tensor host = counts.to(at::kCPU);
    const int64_t* h = host.data_ptr<int64_t>();
    for (int t = 0; t < T; ++t) u[t] = h[t];
  }
  const bool plain = plain_backward();
  std::lock_guard<std::mutex> lock(g_cap_mu);
  drop_dead_records();
  for (int t = 0; t < T; ++t) {
    const Tensor& w = weights[t];
    if (!w.requires_grad()) continue;  // a frozen table gets no gradient
    const int64_t dim = w.size(1);
    const int64_t n = coalesced ? u[t] : lay.cap[t];
    TORCH_CHECK(n >= 0 && n <= lay.cap[t], "coalesced row count outside its capacity");
    Tensor rows = raw_view(rows_all, at::kLong, 8 * lay.rows_off[t], {n}, {1});
    Tensor vals = raw_view(vbuf, w.scalar_type(), lay.val_off[t], {n, dim}, {dim, 1});
    Tensor g = sparse_grad(w, rows, vals, coalesced);
    if (!coalesced) note_capacity_grad(w, rows, vals, raw_view(counts, at::kLong, 8 * t, {1}, {1}));
    if (plain && stores_first_grad(w)) {
      w.mutable_grad() = g;
      g_exact.erase(w.unsafeGetTensorImpl());
      continue;
    }
    if (coalesced) note_exact_grad(w, vals);
    out[t] = std::move(g);
  }
  return out;
}

std::vector<int64_t> table_capacities(int T, TensorList ids, at::IntArrayRef table) {
  std::vector<int64_t> cap(T, 0);
  for (size_t f = 0; f < ids.size(); ++f) cap[table[f]] += ids[f].numel();
  return cap;
}

// The lookup's backward as the modules' autograd runs it: coalesced
// gradients of every table, as sparse COO tensors.
// `sort_in_place`: the keys and payloads are the caller's own (the modules'
// autograd node keeps them private) and may be sorted where they are; the
// operator leaves them as they are, as the forward's outputs they are.
std::vector<std::optional<Tensor>> weight_grads_for(TensorList weights, TensorList ids,
                                                    const c10::List<std::optional<Tensor>>& lengths,
                                                    at::IntArrayRef table, at::IntArrayRef pooling,
                                                    at::IntArrayRef exclude, at::IntArrayRef padding_idx,
                                                    TensorList grads, const Tensor& keys, const Tensor& payload,
                                                    const Tensor& bag_count, const Tensor& offsets, bool coalesced,
                                                    bool sort_in_place) {
  if (!weights.empty() && weights[0].is_cuda()) {
    // ROCm tables: the backward above, called directly (no padding for exact
    // gradients, their counts read before the coalescing reduce is queued)
    std::vector<int64_t> host_counts;
    CoalesceResult r = lookup_backward(weights, ids, lengths, table, pooling, exclude, padding_idx, grads, keys,
                                       payload, bag_count, sort_in_place, !coalesced,
                                       coalesced ? &host_counts : nullptr);
    return weight_grads(weights, r.rows_all, r.vbuf, r.counts, r.layout, coalesced,
                        coalesced ? &host_counts : nullptr);
  }
  // CPU tables: the reference's CPU path registered on the same schema
  static auto op =
      c10::Dispatcher::singleton()
          .findSchemaOrThrow("mdl_hip::grouped_lookup_backward", "")
          .typed<std::tuple<Tensor, Tensor, Tensor>(TensorList, TensorList, const c10::List<std::optional<Tensor>>&,
                                                    at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, at::IntArrayRef,
                                                    TensorList, const Tensor&, const Tensor&, const Tensor&,
                                                    const Tensor&)>();
  auto [rows_all, vbuf, counts] =
      op.call(weights, ids, lengths, table, pooling, exclude, padding_idx, grads, keys, payload, bag_count, offsets);
  const int T = (int)weights.size();
  std::vector<int64_t> esz(T), dims(T);
  for (int t = 0; t < T; ++t) {
    esz[t] = weights[t].element_size();
    dims[t] = weights[t].size(1);
  }
  auto lay = coalesced_layout(esz, dims, table_capacities(T, ids, table));
  return weight_grads(weights, rows_all, vbuf, counts, lay, coalesced);
}

std::vector<std::optional<Tensor>> grouped_lookup_weight_grads(TensorList weights, TensorList ids,
                                                const c10::List<std::optional<Tensor>>& lengths, at::IntArrayRef table,
                                                at::IntArrayRef pooling, at::IntArrayRef exclude,
                                                at::IntArrayRef padding_idx, TensorList grads, const Tensor& keys,
                                                const Tensor& payload, const Tensor& bag_count, const Tensor& offsets,
                                                bool coalesced) {
  return weight_grads_for(weights, ids, lengths, table, pooling, exclude, padding_idx, grads, keys, payload,
                          bag_count, offsets, coalesced, false);
}

// The sparse-gradient mode of the modules' backward, set from Python
// (mdl_amd.library.set_sparse_grad_mode): exact coalesced gradients, or
// capacity-sized ones that need no host read.
std::atomic<bool> g_exact_grads{true};

void set_exact_sparse_grads(bool exact) { g_exact_grads = exact; }

// The modules' grouped lookup as one autograd node in C++ over the tables
// (their only differentiable inputs): the forward calls the lookup below
// autograd, the backward builds every table's sparse gradient with
// grouped_lookup_weight_grads.  No Python runs in the backward, so autograd's
// device thread needs no interpreter lock for it, and the node's state is
// freed without one.
struct GroupedLookupFn : public torch::autograd::Function<GroupedLookupFn> {
  static torch::autograd::variable_list forward(torch::autograd::AutogradContext* ctx, TensorList weights,
                                                const std::vector<Tensor>& ids,
                                                const c10::List<std::optional<Tensor>>& lengths,
                                                at::IntArrayRef table, at::IntArrayRef pooling,
                                                at::IntArrayRef exclude, at::IntArrayRef padding_idx) {
    auto [outputs, keys, payload, bag_count, offsets, err] =
        grouped_lookup_untracked(weights, ids, lengths, table, pooling, exclude, padding_idx, true);
    auto& sd = ctx->saved_data;
    sd["weights"] = weights;
    sd["ids"] = ids;
    sd["lengths"] = lengths;
    sd["table"] = table;
    sd["pooling"] = pooling;
    sd["exclude"] = exclude;
    sd["padding_idx"] = padding_idx;
    sd["keys"] = keys;
    sd["payload"] = payload;
    sd["bag_count"] = bag_count;
    sd["offsets"] = offsets;
    ctx->mark_non_differentiable({err});
    outputs.push_back(err);
    return outputs;
  }

  // One gradient per forward argument: the tables', then none for the ids,
  // lengths and the four per-feature lists.
  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    auto& sd = ctx->saved_data;
    const std::vector<Tensor> weights = sd["weights"].toTensorVector();
    const std::vector<Tensor> ids = sd["ids"].toTensorVector();
    grads.pop_back();  // err
    const std::vector<std::optional<Tensor>> wg = weight_grads_for(
        weights, ids, sd["lengths"].toOptionalTensorList(), sd["table"].toIntVector(), sd["pooling"].toIntVector(),
        sd["exclude"].toIntVector(), sd["padding_idx"].toIntVector(), grads, sd["keys"].toTensor(),
        sd["payload"].toTensor(), sd["bag_count"].toTensor(), sd["offsets"].toTensor(), g_exact_grads.load(), true);
    torch::autograd::variable_list out(weights.size() + 6);
    for (size_t t = 0; t < wg.size(); ++t)
      if (wg[t]) out[t] = *wg[t];
    return out;
  }
};

// A tensor without data of its own: fake or functional (a tracer's), or meta.
bool traced(const Tensor& t) {
  const auto ks = t.key_set();
  return t.is_meta() || ks.has(c10::DispatchKey::Python) || ks.has(c10::DispatchKey::Functionalize);
}

std::vector<Tensor> grouped_lookup_autograd(TensorList weights, TensorList ids,
                                            const c10::List<std::optional<Tensor>>& lengths, at::IntArrayRef table,
                                            at::IntArrayRef pooling, at::IntArrayRef exclude,
                                            at::IntArrayRef padding_idx) {
  TORCH_CHECK_VALUE(!weights.empty() && !ids.empty(), "a grouped lookup needs at least one table and feature");
  if (traced(weights[0]) || traced(ids[0])) {
    // tracers take the public op and its registered autograd, which builds
    // capacity-sized gradients from shapes alone
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("mdl_hip::grouped_lookup", "")
                         .typed<std::tuple<std::vector<Tensor>, Tensor, Tensor, Tensor, Tensor, Tensor>(
                             TensorList, TensorList, const c10::List<std::optional<Tensor>>&, at::IntArrayRef,
                             at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, bool)>();
    auto res = op.call(weights, ids, lengths, table, pooling, exclude, padding_idx, true);
    std::vector<Tensor> out = std::get<0>(res);
    out.push_back(std::get<5>(res));
    return out;
  }
  return GroupedLookupFn::apply(weights, ids.vec(), lengths, table, pooling, exclude, padding_idx);
}

// One parameter's gradient from (rows, values, count): the sequence lookup's.
Tensor capacity_sparse_grad(const Tensor& weight, const Tensor& rows, const Tensor& values, const Tensor& count,
                            bool coalesced) {
  if (coalesced) {
    const int64_t u = count.reshape({-1}).to(at::kCPU).data_ptr<int64_t>()[0];
    TORCH_CHECK(u >= 0 && u <= rows.numel(), "coalesced row count outside its capacity");
    Tensor g = sparse_grad(weight, rows.narrow(0, 0, u), values.narrow(0, 0, u), true);
    std::lock_guard<std::mutex> lock(g_cap_mu);
    drop_dead_records();
    note_exact_grad(weight, g._values());
    return g;
  }
  std::lock_guard<std::mutex> lock(g_cap_mu);
  drop_dead_records();
  note_capacity_grad(weight, rows, values, count.reshape({-1}).narrow(0, 0, 1));
  return sparse_grad(weight, rows, values, false);
}

std::vector<Tensor> capacity_grad_record(const Tensor& param, const Tensor& grad) {
  std::lock_guard<std::mutex> lock(g_cap_mu);
  auto r = find_capacity_grad(param, grad);
  if (!r) return {};
  return {std::get<0>(*r), std::get<1>(*r), std::get<2>(*r)};
}

void forget_capacity_grad(const Tensor& param) {
  std::lock_guard<std::mutex> lock(g_cap_mu);
  g_cap.erase(param.unsafeGetTensorImpl());
}

// optimizer.zero_grad(set_to_none=True) in one call: each parameter's
// gradient reset, as assigning None to .grad does.
void clear_grads_(TensorList params) {
  for (const Tensor& p : params) p.mutable_grad().reset();
}

// ------------------------------------------------------------- row-wise Adagrad --

Tensor row_major_aligned(Tensor t) {
  if (!t.is_contiguous()) t = t.contiguous();
  if (addr(t) % 16 != 0) t = t.clone();
  return t;
}

// One table's share of a grouped update: rows[:count] (count on the device;
// undefined: all rows) of `values` into `w` and its accumulator `a`.
struct UpdateItem {
  const Tensor* w;
  const Tensor* a;
  Tensor rows, values, count;
  double lr;
};

void launch_updates(const at::Device& dev, std::vector<UpdateItem>& items, double eps) {
  const size_t P = items.size();
  if (!P) return;
  const c10::DeviceGuard guard(dev);
  std::vector<mdl_update> ups(P);
  int64_t units = 0;
  for (size_t i = 0; i < P; ++i) {
    UpdateItem& it = items[i];
    const Tensor& w = *it.w;
    const Tensor& a = *it.a;
    require_device(w, "weight");
    TORCH_CHECK_VALUE(w.device() == dev, "one device per grouped update");
    TORCH_CHECK_VALUE(w.dim() == 2 && w.stride(1) == 1, "row-wise Adagrad expects 2D weights with contiguous rows");
    TORCH_CHECK_TYPE(a.scalar_type() == at::kFloat && a.is_contiguous(),
                     "row-wise Adagrad accumulator must be a contiguous float32 tensor");
    if (it.rows.scalar_type() != at::kLong || !it.rows.is_contiguous()) it.rows = it.rows.to(at::kLong).contiguous();
    const auto vt = it.values.scalar_type();
    if ((w.scalar_type() == at::kFloat && vt != at::kFloat) || (vt != at::kFloat && vt != at::kBFloat16))
      it.values = it.values.to(at::kFloat);
    if (!it.values.is_contiguous() || addr(it.values) % 16) it.values = row_major_aligned(it.values);
    mdl_update& u = ups[i];
    u.weight = addr(w);
    u.state = addr(a);
    u.rows = addr(it.rows);
    u.values = addr(it.values);
    u.count = it.count.defined() ? addr(it.count) : 0;
    u.num_rows = w.size(0);
    u.dim = (int32_t)w.size(1);
    u.capacity = it.rows.numel();
    u.weight_stride = w.stride(0);
    u.values_stride = it.values.dim() == 2 && it.values.size(0) ? it.values.stride(0) : w.size(1);
    u.wdtype = dtype_code(w.scalar_type());
    u.vdtype = dtype_code(it.values.scalar_type());
    u.lr = (float)it.lr;
    u.unit_first = units;
    units += (u.capacity + MDL_UPDATE_UNIT - 1) / MDL_UPDATE_UNIT;
  }
  if (units == 0) return;
  Tensor dev_ups = upload_vec(ups, dev);
  check(mdl_grouped_rowwise_adagrad(reinterpret_cast<const mdl_update*>(dev_ups.data_ptr()), ups.data(), (int32_t)P,
                                    (float)eps, nullptr, stream_of(dev)),
        "mdl_grouped_rowwise_adagrad");
}

void grouped_rowwise_adagrad_cuda(TensorList weights, TensorList accumulators, TensorList rows_in,
                                  TensorList values_in, const c10::List<std::optional<Tensor>>& counts,
                                  at::ArrayRef<double> lrs, double eps) {
  const size_t P = weights.size();
  TORCH_CHECK_VALUE(accumulators.size() == P && rows_in.size() == P && values_in.size() == P && counts.size() == P &&
                        lrs.size() == P,
                    "one accumulator, rows, values, count and learning rate per weight");
  if (!P) return;
  std::vector<UpdateItem> items(P);
  for (size_t i = 0; i < P; ++i) {
    const std::optional<Tensor> c = counts.get(i);
    items[i] = UpdateItem{&weights[i], &accumulators[i], rows_in[i], values_in[i],
                          c.has_value() && c->defined() ? *c : Tensor(), lrs[i]};
  }
  launch_updates(weights[0].device(), items, eps);
}

void rowwise_adagrad_cuda(const Tensor& weight, const Tensor& accumulator, const Tensor& rows_in,
                          const Tensor& values_in, double lr, double eps) {
  require_device(weight, "weight");
  TORCH_CHECK_VALUE(weight.dim() == 2, "row-wise Adagrad expects a 2D weight");
  const int64_t n = rows_in.numel();
  if (n == 0) return;
  const c10::DeviceGuard guard(weight.device());
  TORCH_CHECK_TYPE(accumulator.scalar_type() == at::kFloat && accumulator.is_contiguous(),
                   "row-wise Adagrad accumulator must be a contiguous float32 tensor");
  TORCH_CHECK_VALUE(weight.stride(1) == 1, "weight rows must be contiguous");
  Tensor rows = rows_in.to(at::kLong).contiguous();
  Tensor values = values_in;
  if (weight.scalar_type() == at::kFloat && values.scalar_type() != at::kFloat) values = values.to(at::kFloat);
  if (values.scalar_type() != at::kFloat && values.scalar_type() != at::kBFloat16) values = values.to(at::kFloat);
  values = row_major_aligned(values);
  check(mdl_rowwise_adagrad(weight.data_ptr(), dtype_code(weight.scalar_type()), weight.size(0), (int32_t)weight.size(1),
                            weight.stride(0), accumulator.data_ptr<float>(), rows.data_ptr<int64_t>(), n,
                            values.data_ptr(), dtype_code(values.scalar_type()), values.stride(0), (float)lr,
                            (float)eps, nullptr, stream_of(weight.device())),
        "mdl_rowwise_adagrad");
}

// ----------------------------------------------------------- coalescing --

// A one-feature, one-table layout over a stand-in table of num_rows x dim
// (only its row count, dim and dtype are read): the sort/reduce of an
// uncoalesced COO gradient.
std::shared_ptr<Layout> single_table_layout(const Tensor& stand_in, int64_t num_rows, int64_t dim, int32_t dtype,
                                            int64_t padding_idx) {
  auto L = std::make_shared<Layout>();
  mdl_feature d{};
  d.num_rows = num_rows;
  d.dim = (int32_t)dim;
  d.wdtype = dtype;
  d.odtype = dtype;
  d.pooling = MDL_POOL_NONE;
  d.padding_idx = (int32_t)padding_idx;
  L->feats = {d};
  L->row_base = {0};
  L->esz = {dtype == MDL_F32 ? 4 : 2};
  L->dims = {dim};
  L->max_dim = (int)dim;
  KeyGroup g;
  g.lo = 0;
  g.hi = 1;
  g.tables = {0};
  g.rows = num_rows;
  mdl_table r{};
  r.weight = addr(stand_in);
  r.num_rows = num_rows;
  r.dim = (int32_t)dim;
  r.wdtype = dtype;
  r.feature = 0;
  r.gdtype = dtype;
  g.recs = {r};
  g.classes = mdl_table_classes(g.recs.data(), 1);
  L->groups = {g};
  L->sentinel = (uint32_t)num_rows;
  L->key_bits = (int)std::max<int64_t>(1, bit_length(num_rows));
  return L;
}

std::tuple<Tensor, Tensor, Tensor> sparse_coalesce_padded_cuda(const Tensor& indices_in, const Tensor& values_in,
                                                               int64_t num_rows) {
  require_device(values_in, "values");
  const at::Device dev = values_in.device();
  const c10::DeviceGuard guard(dev);
  TORCH_CHECK_VALUE(values_in.dim() == 2, "sparse gradient values must be [n, dim]");
  TORCH_CHECK_VALUE(num_rows > 0 && num_rows < kKeySpace, "num_rows must be in [1, 2^32 - 1)");
  const int64_t n = indices_in.numel();
  const int64_t dim = values_in.size(1);
  Tensor indices = indices_in.to(at::kLong).contiguous();
  Tensor values = row_major_aligned(values_in);
  const int32_t dt = dtype_code(values.scalar_type());
  Tensor stand_in = at::empty({1, dim}, values.options());
  auto L = single_table_layout(stand_in, num_rows, dim, dt, -1);
  auto i32 = at::TensorOptions().dtype(at::kInt).device(dev);
  Tensor keys = at::empty({std::max<int64_t>(n, 1)}, i32), payload = at::empty({std::max<int64_t>(n, 1)}, i32);
  Tensor err = at::zeros({1}, i32);
  if (n)
    check(mdl_sparse_keys(indices.data_ptr<int64_t>(), n, num_rows, 0, 0, -1, reinterpret_cast<uint32_t*>(keys.data_ptr()),
                          reinterpret_cast<uint32_t*>(payload.data_ptr()), L->sentinel, err.data_ptr<int32_t>(),
                          stream_of(dev)),
          "mdl_sparse_keys");
  std::vector<mdl_feature> feats = L->feats;
  feats[0].num_ids = n;
  feats[0].grad = addr(values);
  feats[0].out = addr(values);
  feats[0].out_stride = values.stride(0);
  CoalesceResult r = coalesce_groups(*L, feats, keys, payload, Tensor(), {n}, dev);
  Tensor rows = r.rows_all.narrow(0, 0, n);
  Tensor vals = r.vbuf.narrow(0, 0, r.layout.nbytes[0]).view(values.scalar_type()).view({n, dim});
  return {rows, vals, r.counts};
}

std::tuple<Tensor, Tensor> sparse_coalesce_cuda(const Tensor& indices_in, const Tensor& values_in, int64_t num_rows) {
  require_device(values_in, "values");
  const at::Device dev = values_in.device();
  const c10::DeviceGuard guard(dev);
  TORCH_CHECK_VALUE(values_in.dim() == 2, "sparse gradient values must be [n, dim]");
  TORCH_CHECK_VALUE(num_rows > 0 && num_rows < kKeySpace, "num_rows must be in [1, 2^32 - 1)");
  const int64_t n = indices_in.numel();
  const int64_t dim = values_in.size(1);
  if (n == 0) return {at::empty({0}, indices_in.options().dtype(at::kLong)), values_in.new_empty({0, dim})};
  Tensor indices = indices_in.to(at::kLong).contiguous();
  Tensor values = row_major_aligned(values_in);
  const int32_t dt = dtype_code(values.scalar_type());
  Tensor stand_in = at::empty({1, dim}, values.options());
  auto L = single_table_layout(stand_in, num_rows, dim, dt, -1);
  void* s = stream_of(dev);
  auto i32 = at::TensorOptions().dtype(at::kInt).device(dev);
  Tensor keys = at::empty({n}, i32), payload = at::empty({n}, i32), err = at::zeros({1}, i32);
  check(mdl_sparse_keys(indices.data_ptr<int64_t>(), n, num_rows, 0, 0, -1, reinterpret_cast<uint32_t*>(keys.data_ptr()),
                        reinterpret_cast<uint32_t*>(payload.data_ptr()), L->sentinel, err.data_ptr<int32_t>(), s),
        "mdl_sparse_keys");
  mdl_feature d = L->feats[0];
  d.num_ids = n;
  d.grad = addr(values);
  d.out = addr(values);
  d.out_stride = values.stride(0);
  Tensor meta = upload(&d, sizeof(d), dev);
  Tensor tmeta = upload(L->groups[0].recs.data(), sizeof(mdl_table), dev);
  Tensor ws = workspace(mdl_backward_workspace_bytes(n, 1, (int32_t)dim), dev);
  Tensor urange = at::zeros({2}, at::TensorOptions().dtype(at::kLong).device(dev));
  const auto* td = reinterpret_cast<const mdl_table*>(tmeta.data_ptr());
  uint32_t* k = reinterpret_cast<uint32_t*>(keys.data_ptr());
  uint32_t* p = reinterpret_cast<uint32_t*>(payload.data_ptr());
  check(mdl_backward_count(td, 1, (int32_t)dim, k, p, n, nullptr, L->key_bits, urange.data_ptr<int64_t>(), ws.data_ptr(),
                           (size_t)ws.numel(), s),
        "mdl_backward_count");
  // one read sizes the result, as Tensor.coalesce() does
  Tensor host = at::cat({err.to(at::kLong), urange}).to(at::kCPU);
  const int64_t* h = host.data_ptr<int64_t>();
  TORCH_CHECK_INDEX(h[0] == 0, "sparse gradient rows outside [0, ", num_rows, ")");
  const int64_t u = h[2] - h[1];
  Tensor rows = at::empty({u}, indices.options());
  Tensor summed = at::empty({u, dim}, values.options());
  if (u) {
    const uint64_t a[2] = {addr(rows), addr(summed)};
    Tensor ad = upload(a, sizeof(a), dev);
    const auto* ap = reinterpret_cast<const uint64_t*>(ad.data_ptr());
    check(mdl_backward_coalesce(reinterpret_cast<const mdl_feature*>(meta.data_ptr()), 1, td, 1, (int32_t)dim, k, p, n,
                                L->key_bits, nullptr, urange.data_ptr<int64_t>(), ap, ap + 1, ws.data_ptr(),
                                (size_t)ws.numel(), L->groups[0].classes, s),
          "mdl_backward_coalesce");
  }
  return {rows, summed};
}

// ------------------------------------------------------------- optimizer --
//
// ShardedRowWiseAdagrad.step for a parameter group (src/optim.py:299-377):
// every parameter with a gradient is checked, its CPU step count advanced and
// its learning rate decayed here; the device parameters are then updated by
// one grouped launch per device, the CPU ones by the reference's CPU branch
// (:359-376).

void cpu_branch(const Tensor& param, const Tensor& acc, const Tensor& rows, const Tensor& values, double lr,
                double eps) {
  if (rows.numel() == 0) return;
  Tensor sv = values.scalar_type() == at::kFloat ? values : values.to(at::kFloat);
  acc.index_add_(0, rows, sv.square().mean(1));
  Tensor den = acc.index_select(0, rows).sqrt_().add_(eps).unsqueeze(1);
  Tensor update = sv / den;
  if (update.scalar_type() != param.scalar_type()) update = update.to(param.scalar_type());
  param.index_add_(0, rows, update, -lr);
}

void rowwise_adagrad_step(TensorList params, TensorList sums, TensorList steps,
                          const c10::List<std::optional<Tensor>>& grads, double lr, double lr_decay, double eps) {
  const size_t P = params.size();
  TORCH_CHECK_VALUE(sums.size() == P && steps.size() == P && grads.size() == P,
                    "one accumulator, step count and gradient per parameter");
  std::vector<std::pair<at::Device, std::vector<UpdateItem>>> batches;
  struct HostItem {
    size_t i;
    Tensor grad;
    double lr;
  };
  std::vector<HostItem> host_items;
  std::unique_lock<std::mutex> lock(g_cap_mu);
  for (size_t i = 0; i < P; ++i) {
    const std::optional<Tensor> og = grads.get(i);
    if (!og.has_value() || !og->defined()) continue;  // skipped before the step count, as the reference does
    const Tensor& grad = *og;
    TORCH_CHECK(grad.is_sparse() && grad.layout() == at::kSparse,
                "ShardedRowWiseAdagrad expects one-dimensional row-sparse COO gradients");
    const auto* sp = at::sparse::get_sparse_impl(grad);
    TORCH_CHECK(sp->sparse_dim() == 1 && sp->dense_dim() == 1,
                "ShardedRowWiseAdagrad expects one sparse row dimension and one dense dimension");
    const Tensor& step = steps[i];
    TORCH_CHECK(step.device().is_cpu() && step.scalar_type() == at::kDouble && step.numel() == 1,
                "ShardedRowWiseAdagrad step counts are 0-d float64 CPU tensors");
    double* stp = step.data_ptr<double>();
    const double k = *stp + 1.0;
    *stp = k;
    const double clr = lr_decay == 0.0 ? lr : lr / (1.0 + (k - 1.0) * lr_decay);
    const Tensor& p = params[i];
    if (!p.is_cuda()) {
      host_items.push_back(HostItem{i, grad, clr});
      continue;
    }
    UpdateItem it{&p, &sums[i], Tensor(), Tensor(), Tensor(), clr};
    auto rec = find_capacity_grad(p, grad);
    if (rec) {
      std::tie(it.rows, it.values, it.count) = *rec;
      g_cap.erase(p.unsafeGetTensorImpl());
    } else {
      const Tensor& idx = sp->indices();
      const int64_t nnz = sp->nnz();
      Tensor rows = raw_view(idx, at::kLong, 0, {nnz}, {idx.stride(1)});
      if (sp->coalesced()) {
        it.rows = rows;
        it.values = sp->values();
      } else {
        std::tie(it.rows, it.values, it.count) = sparse_coalesce_padded_cuda(rows, sp->values(), p.size(0));
      }
    }
    auto b = std::find_if(batches.begin(), batches.end(), [&](const auto& e) { return e.first == p.device(); });
    if (b == batches.end()) {
      batches.emplace_back(p.device(), std::vector<UpdateItem>());
      b = batches.end() - 1;
      b->second.reserve(P);
    }
    b->second.push_back(std::move(it));
  }
  lock.unlock();
  for (auto& [dev, items] : batches) launch_updates(dev, items, eps);
  for (const HostItem& h : host_items) {
    Tensor g = h.grad.coalesce();
    cpu_branch(params[h.i], sums[h.i], g._indices()[0], g._values(), h.lr, eps);
  }
}

// ------------------------------------------------------------------ clip --
//
// The trainer's sparse clip (src/train.py:5730-5826) over parameter lists in
// one call: every gradient's values -- a capacity-sized gradient's values as
// they are (its padding rows hold zeros), a coalesced one's as they are,
// any other sparse gradient coalesced exactly (one host read) and stored
// back as the parameter's gradient, a dense gradient as it is -- then one
// multi-tensor sum of squares per list, min(max_norm / (norm + 1e-6), 1) on
// the device and one multi-tensor scale of every gradient in its own dtype.
// Returns the pre-clip norm (0-d fp32 on the device).

// A gradient's values for the clip, and for a capacity-sized gradient the
// device count of its live rows (the clip then stops at them).
struct ClipValues {
  Tensor values;
  Tensor live_rows;  // undefined: all rows count
};

std::vector<ClipValues> clip_values(TensorList params) {
  std::vector<ClipValues> out;
  out.reserve(params.size());
  for (const Tensor& p : params) {
    const Tensor& g = p.grad();
    if (!g.defined()) continue;
    require_device(g, "gradient");
    if (!g.is_sparse()) {
      out.push_back({g, Tensor()});
      continue;
    }
    std::optional<std::tuple<Tensor, Tensor, Tensor>> rec;
    {
      std::lock_guard<std::mutex> lock(g_cap_mu);
      rec = find_capacity_grad(p, g);
    }
    const auto* sp = at::sparse::get_sparse_impl(g);
    if (rec) {
      out.push_back({std::get<1>(*rec), std::get<2>(*rec)});
    } else if (sp->coalesced()) {
      out.push_back({sp->values(), Tensor()});
    } else {
      const Tensor& idx = sp->indices();
      Tensor rows = raw_view(idx, at::kLong, 0, {sp->nnz()}, {idx.stride(1)});
      auto [urows, vals] = sparse_coalesce_cuda(rows, sp->values(), p.size(0));
      p.mutable_grad() = sparse_grad(p, urows, vals, true);
      out.push_back({vals, Tensor()});
    }
  }
  return out;
}

std::vector<mdl_span> spans_of(const std::vector<ClipValues>& vs) {
  std::vector<mdl_span> spans;
  spans.reserve(vs.size());
  for (const ClipValues& v : vs) {
    const Tensor& t = v.values;
    if (!t.numel()) continue;
    TORCH_CHECK_VALUE(t.is_contiguous(), "gradients to clip must be contiguous");
    mdl_span sp{};
    sp.data = addr(t);
    sp.numel = t.numel();
    sp.dtype = dtype_code(t.scalar_type());
    if (v.live_rows.defined()) {
      sp.row_elems = (int32_t)(t.dim() > 1 ? t.size(1) : 1);
      sp.live_rows = v.live_rows.data_ptr<int64_t>();
    }
    spans.push_back(sp);
  }
  return spans;
}

Tensor clip_sparse_grad_norm_(TensorList replicated, TensorList sharded, double max_norm) {
  const Tensor* first = nullptr;
  for (TensorList l : {replicated, sharded})
    if (!first && !l.empty()) first = &l[0];
  if (!first) return at::zeros({}, at::TensorOptions().dtype(at::kFloat));
  const at::Device dev = first->device();
  require_device(*first, "parameter");
  const c10::DeviceGuard guard(dev);
  void* s = stream_of(dev);
  const std::vector<ClipValues> rv = clip_values(replicated), sv = clip_values(sharded);
  const std::vector<mdl_span> rs = spans_of(rv), ss = spans_of(sv);
  // one upload: both lists' spans
  std::vector<mdl_span> all(rs);
  all.insert(all.end(), ss.begin(), ss.end());
  Tensor spans_dev = upload_vec(all, dev);
  const auto* sd = reinterpret_cast<const mdl_span*>(spans_dev.data_ptr());
  auto f32 = at::TensorOptions().dtype(at::kFloat).device(dev);
  Tensor sumsq = at::empty({2}, f32), norm = at::empty({1}, f32), coef = at::empty({1}, f32);
  const size_t wsb = mdl_sumsq_workspace_bytes((int32_t)std::max(rs.size(), ss.size()));
  Tensor ws = workspace(wsb, dev);
  check(mdl_sumsq(rs.empty() ? nullptr : sd, (int32_t)rs.size(), sumsq.data_ptr<float>(), ws.data_ptr(), wsb, s),
        "mdl_sumsq");
  check(mdl_sumsq(ss.empty() ? nullptr : sd + rs.size(), (int32_t)ss.size(), sumsq.data_ptr<float>() + 1,
                  ws.data_ptr(), wsb, s),
        "mdl_sumsq");
  check(mdl_clip_coef(sumsq.data_ptr<float>(), 2, (float)max_norm, norm.data_ptr<float>(), coef.data_ptr<float>(), s),
        "mdl_clip_coef");
  if (!all.empty()) check(mdl_scale(sd, (int32_t)all.size(), coef.data_ptr<float>(), s), "mdl_scale");
  return norm.reshape({});
}

// ------------------------------------------------------------- bucketing --

std::tuple<Tensor, Tensor> bucketize_cuda(const Tensor& raw_in, const std::optional<Tensor>& valid_in,
                                          int64_t num_buckets, c10::string_view mode, bool validate_nonzero) {
  require_device(raw_in, "raw ids");
  TORCH_CHECK_TYPE(raw_in.scalar_type() == at::kLong, "raw ids must be torch.int64");
  TORCH_CHECK_VALUE(mode == "pre_hashed" || mode == "mod", "mode must be pre_hashed or mod");
  const c10::DeviceGuard guard(raw_in.device());
  Tensor raw = raw_in.contiguous();
  Tensor out = at::empty_like(raw);
  Tensor err = at::zeros({1}, raw.options().dtype(at::kInt));
  Tensor valid;
  if (valid_in.has_value() && valid_in->defined()) valid = valid_in->to(raw.device(), at::kByte).contiguous();
  check(mdl_bucketize(raw.data_ptr<int64_t>(), valid.defined() ? valid.data_ptr<uint8_t>() : nullptr, raw.numel(),
                      num_buckets, mode == "pre_hashed" ? MDL_BUCKET_PRE_HASHED : MDL_BUCKET_MOD,
                      validate_nonzero ? 1 : 0, out.data_ptr<int64_t>(), err.data_ptr<int32_t>(),
                      stream_of(raw.device())),
        "mdl_bucketize");
  return {out, err};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> bag_truncate_cuda(const Tensor& values_in, const Tensor& offsets_in,
                                                             const std::optional<Tensor>& valid_in,
                                                             const std::optional<Tensor>& row_valid_in,
                                                             int64_t max_length, c10::string_view truncation,
                                                             c10::string_view bucket, int64_t num_buckets,
                                                             bool validate_nonzero) {
  require_device(values_in, "list values");
  TORCH_CHECK_TYPE(values_in.scalar_type() == at::kLong && offsets_in.scalar_type() == at::kLong,
                   "list values and offsets must be torch.int64");
  int32_t bmode = -1;
  if (bucket == "none") bmode = MDL_BUCKET_NONE;
  else if (bucket == "pre_hashed") bmode = MDL_BUCKET_PRE_HASHED;
  else if (bucket == "mod") bmode = MDL_BUCKET_MOD;
  TORCH_CHECK_VALUE(bmode >= 0, "bucket must be one of ['mod', 'none', 'pre_hashed']");
  TORCH_CHECK_VALUE(truncation == "head" || truncation == "tail", "unsupported list truncation '",
                    std::string(truncation), "'");
  const at::Device dev = values_in.device();
  const c10::DeviceGuard guard(dev);
  Tensor values = values_in.contiguous();
  Tensor offsets = offsets_in.to(dev).contiguous();
  const int64_t rows = offsets.numel() - 1;
  TORCH_CHECK_VALUE(rows >= 0, "list offsets need at least one entry");
  Tensor valid, row_valid;
  if (valid_in.has_value() && valid_in->defined()) valid = valid_in->to(dev, at::kByte).contiguous();
  if (row_valid_in.has_value() && row_valid_in->defined()) row_valid = row_valid_in->to(dev, at::kByte).contiguous();
  const int64_t n_in = values.numel();
  auto i64 = at::TensorOptions().dtype(at::kLong).device(dev);
  Tensor ids = at::empty({n_in}, i64), lengths = at::empty({rows}, i64), out_offsets = at::empty({rows + 1}, i64);
  Tensor err = at::zeros({1}, at::TensorOptions().dtype(at::kInt).device(dev));
  Tensor ws = workspace(mdl_bag_truncate_workspace_bytes(rows), dev);
  check(mdl_bag_truncate(offsets.data_ptr<int64_t>(), row_valid.defined() ? row_valid.data_ptr<uint8_t>() : nullptr,
                         rows, n_in ? values.data_ptr<int64_t>() : nullptr,
                         valid.defined() ? valid.data_ptr<uint8_t>() : nullptr, n_in, max_length < 0 ? -1 : max_length,
                         truncation == "head" ? MDL_TRUNCATE_HEAD : MDL_TRUNCATE_TAIL, bmode, num_buckets,
                         validate_nonzero ? 1 : 0, rows ? lengths.data_ptr<int64_t>() : nullptr,
                         out_offsets.data_ptr<int64_t>(), n_in ? ids.data_ptr<int64_t>() : nullptr, n_in,
                         err.data_ptr<int32_t>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(dev)),
        "mdl_bag_truncate");
  return {ids, lengths, out_offsets, err};
}

Tensor lengths_to_offsets_cuda(const Tensor& lengths_in) {
  require_device(lengths_in, "lengths");
  const c10::DeviceGuard guard(lengths_in.device());
  Tensor lengths = lengths_in.to(at::kLong).contiguous();
  const int64_t n = lengths.numel();
  Tensor offsets = at::empty({n + 1}, lengths.options());
  Tensor ws = workspace(mdl_offsets_workspace_bytes(n), lengths.device());
  check(mdl_lengths_to_offsets(lengths.data_ptr<int64_t>(), n, offsets.data_ptr<int64_t>(), ws.data_ptr(),
                               (size_t)ws.numel(), stream_of(lengths.device())),
        "mdl_lengths_to_offsets");
  return offsets;
}

// ------------------------------------------------------------- sequences --

mdl_feature sequence_record(const Tensor& weight, int64_t padding_idx) {
  mdl_feature d{};
  d.weight = addr(weight);
  d.num_rows = weight.size(0);
  d.dim = (int32_t)weight.size(1);
  d.wdtype = dtype_code(weight.scalar_type());
  d.odtype = d.wdtype;
  d.pooling = MDL_POOL_NONE;
  d.padding_idx = (int32_t)padding_idx;
  d.out_stride = weight.size(1);
  return d;
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> sequence_lookup_cuda(const Tensor& weight, const Tensor& ids_in,
                                                                       const Tensor& lengths_in, int64_t out_len,
                                                                       bool newest_first, int64_t padding_idx,
                                                                       bool need_backward) {
  require_device(weight, "embedding weight");
  require_device(ids_in, "sequence ids");
  TORCH_CHECK_TYPE(ids_in.scalar_type() == at::kLong, "sharded embedding indices must be torch.long");
  TORCH_CHECK_VALUE(ids_in.dim() == 2, "sequence ids must be [batch, length]");
  TORCH_CHECK_VALUE(weight.dim() == 2 && weight.stride(1) == 1 && weight.stride(0) == weight.size(1),
                    "embedding weights must be contiguous [rows, dim] tensors");
  TORCH_CHECK_VALUE(out_len >= 0, "the window length must be non-negative");
  TORCH_CHECK_VALUE(weight.size(0) < kKeySpace, "a table of a grouped lookup holds fewer than 2^32 - 1 rows");
  const at::Device dev = weight.device();
  const c10::DeviceGuard guard(dev);
  const int64_t B = ids_in.size(0), in_len = ids_in.size(1), dim = weight.size(1);
  Tensor ids = ids_in.contiguous();
  Tensor lengths = lengths_in.to(dev, at::kLong).contiguous();
  Tensor out = at::empty({B, out_len, dim}, weight.options());
  Tensor mask = at::empty({B, out_len}, weight.options().dtype(at::kBool));
  mdl_feature d = sequence_record(weight, padding_idx);
  const int64_t n = B * out_len;
  auto i32 = at::TensorOptions().dtype(at::kInt).device(dev);
  Tensor keys = at::empty({0}, i32), payload = at::empty({0}, i32);
  if (need_backward) {
    keys = at::empty({std::max<int64_t>(n, 1)}, i32);
    payload = at::empty({std::max<int64_t>(n, 1)}, i32);
  }
  Tensor err = at::zeros({1}, i32);
  check(mdl_sequence_forward(&d, ids.data_ptr<int64_t>(), lengths.data_ptr<int64_t>(), B, in_len, out_len,
                             newest_first ? MDL_SEQ_NEWEST_TO_OLDEST : MDL_SEQ_OLDEST_TO_NEWEST, out.data_ptr(),
                             reinterpret_cast<uint8_t*>(mask.data_ptr()),
                             need_backward ? reinterpret_cast<uint32_t*>(keys.data_ptr()) : nullptr,
                             need_backward ? reinterpret_cast<uint32_t*>(payload.data_ptr()) : nullptr, nullptr,
                             (uint32_t)weight.size(0), err.data_ptr<int32_t>(), stream_of(dev)),
        "mdl_sequence_forward");
  return {out, mask, keys, payload, err};
}

std::tuple<Tensor, Tensor, Tensor> sequence_lookup_backward_cuda(const Tensor& weight, const Tensor& ids,
                                                                 const Tensor& lengths, int64_t out_len,
                                                                 bool newest_first, int64_t padding_idx,
                                                                 const Tensor& grad, const Tensor& keys_in,
                                                                 const Tensor& payload_in) {
  require_device(weight, "embedding weight");
  const at::Device dev = weight.device();
  const c10::DeviceGuard guard(dev);
  const int64_t n = ids.size(0) * out_len;
  const int64_t dim = weight.size(1);
  TORCH_CHECK_VALUE(keys_in.numel() >= n && payload_in.numel() >= n,
                    "sequence sort keys hold one entry per window position (batch * out_len)");
  Tensor keys = keys_in.clone(), payload = payload_in.clone();
  Tensor stand_in = weight;
  auto L = single_table_layout(stand_in, weight.size(0), dim, dtype_code(weight.scalar_type()), padding_idx);
  std::vector<mdl_feature> feats = {sequence_record(weight, padding_idx)};
  feats[0].num_ids = n;
  Tensor g = grad;
  if (g.scalar_type() != weight.scalar_type()) g = g.to(weight.scalar_type());
  g = g.reshape({-1, dim});
  TORCH_CHECK_VALUE(g.size(0) == n, "the window gradient must be [batch, out_len, dim]");
  if (g.stride(-1) != 1 || addr(g) % 16 || (g.stride(0) * g.element_size()) % 16) g = row_major_aligned(g.contiguous());
  feats[0].grad = addr(g);
  feats[0].out = addr(g);
  feats[0].out_stride = g.stride(0);
  CoalesceResult r = coalesce_groups(*L, feats, keys, payload, Tensor(), {n}, dev);
  Tensor rows = r.rows_all.narrow(0, 0, n);
  Tensor vals = r.vbuf.narrow(0, 0, r.layout.nbytes[0]).view(weight.scalar_type()).view({n, dim});
  return {rows, vals, r.counts};
}

// ------------------------------------------------------- the fused step --
//
// SparseStep / SequenceStep launches: descriptors, chunks, tables and the
// workspace are the caller's device tensors, built once per layout; the
// weights and accumulators they address are named so the schema states
// what the step mutates.

template <typename T>
T* at_offset(const Tensor& t, int64_t elements) {
  return reinterpret_cast<T*>(static_cast<uint8_t*>(t.data_ptr()) + elements * (int64_t)sizeof(T));
}

void packed_forward_(const Tensor& features, int64_t feature_offset, int64_t num_features, const Tensor& chunks,
                     int64_t num_chunks, const Tensor& ids, int64_t num_ids, const std::optional<Tensor>& offsets,
                     const std::optional<Tensor>& keys, const std::optional<Tensor>& payload, int64_t key_offset,
                     const std::optional<Tensor>& key_origin, int64_t key_origin_offset, int64_t sentinel,
                     const std::optional<Tensor>& bag_count, const Tensor& error_count, TensorList outputs,
                     int64_t classes) {
  (void)outputs;
  const at::Device dev = features.device();
  const c10::DeviceGuard guard(dev);
  check(mdl_forward(at_offset<mdl_feature>(features, feature_offset), (int32_t)num_features,
                    reinterpret_cast<const mdl_chunk*>(chunks.data_ptr()), num_chunks, ids.data_ptr<int64_t>(), num_ids,
                    ptr_or_null<int64_t>(offsets),
                    keys.has_value() && keys->defined() ? at_offset<uint32_t>(*keys, key_offset) : nullptr,
                    payload.has_value() && payload->defined() ? at_offset<uint32_t>(*payload, key_offset) : nullptr,
                    key_origin.has_value() && key_origin->defined() ? at_offset<int64_t>(*key_origin, key_origin_offset)
                                                                    : nullptr,
                    (uint32_t)sentinel, ptr_or_null<float>(bag_count), error_count.data_ptr<int32_t>(),
                    (uint32_t)classes, stream_of(dev)),
        "mdl_forward");
}

void backward_sort_(const Tensor& tables, int64_t num_tables, const Tensor& keys, const Tensor& payload,
                    int64_t num_entries, const std::optional<Tensor>& count, int64_t count_offset, int64_t max_dim,
                    int64_t key_bits, const Tensor& ws) {
  const at::Device dev = keys.device();
  const c10::DeviceGuard guard(dev);
  check(mdl_backward_sort(reinterpret_cast<const mdl_table*>(tables.data_ptr()), (int32_t)num_tables, (int32_t)max_dim,
                          reinterpret_cast<uint32_t*>(keys.data_ptr()), reinterpret_cast<uint32_t*>(payload.data_ptr()),
                          num_entries,
                          count.has_value() && count->defined() ? at_offset<int64_t>(*count, count_offset) : nullptr,
                          (int32_t)key_bits, ws.data_ptr(), (size_t)ws.numel(), stream_of(dev)),
        "mdl_backward_sort");
}

void backward_apply_(TensorList weights, TensorList accumulators, const Tensor& features, int64_t num_features,
                     const Tensor& tables, int64_t num_tables, const Tensor& keys, const Tensor& payload,
                     int64_t num_entries, const std::optional<Tensor>& bag_count, const std::optional<Tensor>& grad_scale,
                     const Tensor& ws, int64_t max_dim, int64_t key_bits, int64_t classes, double lr, double eps) {
  (void)weights;
  (void)accumulators;
  const at::Device dev = keys.device();
  const c10::DeviceGuard guard(dev);
  check(mdl_backward_apply(reinterpret_cast<const mdl_feature*>(features.data_ptr()), (int32_t)num_features,
                           reinterpret_cast<const mdl_table*>(tables.data_ptr()), (int32_t)num_tables, (int32_t)max_dim,
                           reinterpret_cast<uint32_t*>(keys.data_ptr()), reinterpret_cast<uint32_t*>(payload.data_ptr()),
                           num_entries, (int32_t)key_bits, ptr_or_null<float>(bag_count), (float)lr, (float)eps,
                           ptr_or_null<float>(grad_scale), ws.data_ptr(), (size_t)ws.numel(), (uint32_t)classes,
                           stream_of(dev)),
        "mdl_backward_apply");
}

void fused_backward_rowwise_adagrad_(TensorList weights, TensorList accumulators, const Tensor& features,
                                     int64_t num_features, const Tensor& tables, int64_t num_tables, const Tensor& keys,
                                     const Tensor& payload, int64_t num_entries, const std::optional<Tensor>& count,
                                     int64_t count_offset, const std::optional<Tensor>& bag_count,
                                     const std::optional<Tensor>& grad_scale, const Tensor& ws, int64_t max_dim,
                                     int64_t key_bits, int64_t classes, double lr, double eps) {
  (void)weights;
  (void)accumulators;
  const at::Device dev = keys.device();
  const c10::DeviceGuard guard(dev);
  check(mdl_backward_adagrad(reinterpret_cast<const mdl_feature*>(features.data_ptr()), (int32_t)num_features,
                             reinterpret_cast<const mdl_table*>(tables.data_ptr()), (int32_t)num_tables, (int32_t)max_dim,
                             reinterpret_cast<uint32_t*>(keys.data_ptr()), reinterpret_cast<uint32_t*>(payload.data_ptr()),
                             num_entries,
                             count.has_value() && count->defined() ? at_offset<int64_t>(*count, count_offset) : nullptr,
                             (int32_t)key_bits, ptr_or_null<float>(bag_count), (float)lr, (float)eps,
                             ptr_or_null<float>(grad_scale), ws.data_ptr(), (size_t)ws.numel(), (uint32_t)classes,
                             stream_of(dev)),
        "mdl_backward_adagrad");
}

void backward_sumsq_(const Tensor& features, int64_t num_features, const Tensor& tables, int64_t num_tables,
                     const Tensor& keys, const Tensor& payload, int64_t num_entries,
                     const std::optional<Tensor>& bag_count, const Tensor& sumsq, int64_t slot, const Tensor& ws,
                     int64_t max_dim, int64_t key_bits, int64_t classes) {
  const at::Device dev = keys.device();
  const c10::DeviceGuard guard(dev);
  check(mdl_backward_sumsq(reinterpret_cast<const mdl_feature*>(features.data_ptr()), (int32_t)num_features,
                           reinterpret_cast<const mdl_table*>(tables.data_ptr()), (int32_t)num_tables, (int32_t)max_dim,
                           reinterpret_cast<uint32_t*>(keys.data_ptr()), reinterpret_cast<uint32_t*>(payload.data_ptr()),
                           num_entries, (int32_t)key_bits, ptr_or_null<float>(bag_count), at_offset<float>(sumsq, slot),
                           ws.data_ptr(), (size_t)ws.numel(), (uint32_t)classes, stream_of(dev)),
        "mdl_backward_sumsq");
}

void clip_coefficient_(const Tensor& sumsq, int64_t count, double max_norm, const Tensor& total_norm,
                       const Tensor& coef) {
  const at::Device dev = sumsq.device();
  const c10::DeviceGuard guard(dev);
  TORCH_CHECK_VALUE(sumsq.scalar_type() == at::kFloat && sumsq.is_contiguous() && sumsq.numel() >= count,
                    "squared norms are a contiguous float32 tensor");
  check(mdl_clip_coef(sumsq.data_ptr<float>(), (int32_t)count, (float)max_norm, total_norm.data_ptr<float>(),
                      coef.data_ptr<float>(), stream_of(dev)),
        "mdl_clip_coef");
}

}  // namespace mdl_torch

// ---------------------------------------------------------- registration --

TORCH_LIBRARY(mdl_hip, m) {
  using namespace mdl_torch;
  // Operators with a CPU kernel (registered from Python, the reference's CPU
  // semantics) and a fake kernel: the path's public ops.
  m.def("bucketize(Tensor raw, Tensor? valid, int num_buckets, str mode, bool validate_nonzero) -> (Tensor, Tensor)");
  m.def("bag_truncate(Tensor values, Tensor offsets, Tensor? valid, Tensor? row_valid, int max_length, "
        "str truncation, str bucket, int num_buckets, bool validate_nonzero) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("lengths_to_offsets(Tensor lengths) -> Tensor");
  m.def("grouped_lookup(Tensor[] weights, Tensor[] ids, Tensor?[] lengths, int[] table, int[] pooling, "
        "int[] exclude, int[] padding_idx, bool need_backward) -> (Tensor[], Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("grouped_lookup_untracked(Tensor[] weights, Tensor[] ids, Tensor?[] lengths, int[] table, int[] pooling, "
        "int[] exclude, int[] padding_idx, bool need_backward) -> (Tensor[], Tensor, Tensor, Tensor, Tensor, Tensor)",
        &grouped_lookup_untracked);
  m.def("grouped_lookup_autograd(Tensor[] weights, Tensor[] ids, Tensor?[] lengths, int[] table, int[] pooling, "
        "int[] exclude, int[] padding_idx) -> Tensor[]",
        &grouped_lookup_autograd);
  m.def("set_exact_sparse_grads(bool exact) -> ()", &set_exact_sparse_grads);
  m.def("grouped_lookup_backward(Tensor[] weights, Tensor[] ids, Tensor?[] lengths, int[] table, int[] pooling, "
        "int[] exclude, int[] padding_idx, Tensor[] grads, Tensor keys, Tensor payload, Tensor bag_count, "
        "Tensor offsets) -> (Tensor, Tensor, Tensor)");
  m.def("sequence_lookup(Tensor weight, Tensor ids, Tensor lengths, int out_len, bool newest_first, "
        "int padding_idx, bool need_backward) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("sequence_lookup_backward(Tensor weight, Tensor ids, Tensor lengths, int out_len, bool newest_first, "
        "int padding_idx, Tensor grad, Tensor keys, Tensor payload) -> (Tensor, Tensor, Tensor)");
  m.def("sparse_coalesce(Tensor indices, Tensor values, int num_rows) -> (Tensor, Tensor)");
  m.def("sparse_coalesce_padded(Tensor indices, Tensor values, int num_rows) -> (Tensor, Tensor, Tensor)");
  m.def("rowwise_adagrad_(Tensor(a!) weight, Tensor(b!) accumulator, Tensor rows, Tensor values, float lr, "
        "float eps) -> ()");
  m.def("grouped_rowwise_adagrad_(Tensor(a!)[] weights, Tensor(b!)[] accumulators, Tensor[] rows, "
        "Tensor[] values, Tensor?[] counts, float[] lrs, float eps) -> ()");
  // The modules' autograd and optimizer: whole steps of host work in one call
  // (registered for every backend; CPU tensors take the reference's CPU paths).
  m.def("grouped_lookup_weight_grads(Tensor[] weights, Tensor[] ids, Tensor?[] lengths, int[] table, "
        "int[] pooling, int[] exclude, int[] padding_idx, Tensor[] grads, Tensor keys, Tensor payload, "
        "Tensor bag_count, Tensor offsets, bool coalesced) -> Tensor?[]",
        &grouped_lookup_weight_grads);
  m.def("capacity_sparse_grad(Tensor weight, Tensor rows, Tensor values, Tensor count, bool coalesced) -> Tensor",
        &capacity_sparse_grad);
  m.def("capacity_grad_record(Tensor param, Tensor grad) -> Tensor[]", &capacity_grad_record);
  m.def("lookup_order(Tensor[] weights, int[] table) -> int[]", &lookup_order);
  m.def("forget_capacity_grad(Tensor param) -> ()", &forget_capacity_grad);
  m.def("clear_grads_(Tensor[] params) -> ()", &clear_grads_);
  m.def("rowwise_adagrad_step_(Tensor(a!)[] params, Tensor(b!)[] sums, Tensor(c!)[] steps, Tensor?[] grads, "
        "float lr, float lr_decay, float eps) -> ()",
        &rowwise_adagrad_step);
  // The fused step of a fixed layout (SparseStep / SequenceStep): device
  // descriptors built once, launches only.
  m.def("packed_forward_(Tensor features, int feature_offset, int num_features, Tensor chunks, int num_chunks, "
        "Tensor ids, int num_ids, Tensor? offsets, Tensor(a!)? keys, Tensor(b!)? payload, int key_offset, "
        "Tensor? key_origin, int key_origin_offset, int sentinel, Tensor(c!)? bag_count, Tensor(d!) error_count, "
        "Tensor(e!)[] outputs, int classes) -> ()",
        &packed_forward_);
  m.def("backward_sort_(Tensor tables, int num_tables, Tensor(a!) keys, Tensor(b!) payload, int num_entries, "
        "Tensor? count, int count_offset, int max_dim, int key_bits, Tensor(c!) workspace) -> ()",
        &backward_sort_);
  m.def("backward_apply_(Tensor(a!)[] weights, Tensor(b!)[] accumulators, Tensor features, int num_features, "
        "Tensor tables, int num_tables, Tensor keys, Tensor payload, int num_entries, Tensor? bag_count, "
        "Tensor? grad_scale, Tensor(c!) workspace, int max_dim, int key_bits, int classes, float lr, float eps) -> ()",
        &backward_apply_);
  m.def("fused_backward_rowwise_adagrad_(Tensor(a!)[] weights, Tensor(b!)[] accumulators, Tensor features, "
        "int num_features, Tensor tables, int num_tables, Tensor(c!) keys, Tensor(d!) payload, int num_entries, "
        "Tensor? count, int count_offset, Tensor? bag_count, Tensor? grad_scale, Tensor(e!) workspace, "
        "int max_dim, int key_bits, int classes, float lr, float eps) -> ()",
        &fused_backward_rowwise_adagrad_);
  m.def("backward_sumsq_(Tensor features, int num_features, Tensor tables, int num_tables, Tensor keys, "
        "Tensor payload, int num_entries, Tensor? bag_count, Tensor(a!) sumsq, int slot, Tensor(b!) workspace, "
        "int max_dim, int key_bits, int classes) -> ()",
        &backward_sumsq_);
  m.def("clip_coefficient_(Tensor sumsq, int count, float max_norm, Tensor(a!) total_norm, Tensor(b!) coef) -> ()",
        &clip_coefficient_);
  // The trainer's sparse clip over parameter lists (their gradients scaled
  // in place, some coalesced and stored back).
  m.def("clip_sparse_grad_norm_(Tensor(a!)[] replicated, Tensor(b!)[] sharded, float max_norm) -> Tensor",
        &clip_sparse_grad_norm_);
}

TORCH_LIBRARY_IMPL(mdl_hip, CUDA, m) {
  using namespace mdl_torch;
  m.impl("bucketize", &bucketize_cuda);
  m.impl("bag_truncate", &bag_truncate_cuda);
  m.impl("lengths_to_offsets", &lengths_to_offsets_cuda);
  m.impl("grouped_lookup", &grouped_lookup_cuda);
  m.impl("grouped_lookup_backward", &grouped_lookup_backward_cuda);
  m.impl("sequence_lookup", &sequence_lookup_cuda);
  m.impl("sequence_lookup_backward", &sequence_lookup_backward_cuda);
  m.impl("sparse_coalesce", &sparse_coalesce_cuda);
  m.impl("sparse_coalesce_padded", &sparse_coalesce_padded_cuda);
  m.impl("rowwise_adagrad_", &rowwise_adagrad_cuda);
  m.impl("grouped_rowwise_adagrad_", &grouped_rowwise_adagrad_cuda);
}
