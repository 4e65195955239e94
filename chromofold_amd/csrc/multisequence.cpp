// multisequence.cpp — host bookkeeping of sequences over shared, refcounted immutable pages (cf_multisequence_*).
//
// Semantics follow reference src/multisequence_cache.cpp: config check :63-68; page acquire/release with the
// shared-page and pending-reclamation counters :99-125; page-order validation :133-145; audit :147-175;
// create :194-213; copy of the pages (and active range) inside [begin, end) :215-283; removal of the whole
// sequence or of whole pages + an active suffix :285-353; shift of whole pages + the active range :355-393;
// contiguous appends inside one active page :395-427; attention validation then refusal (no dense fallback)
// :429-451; speculative begin / commit / rollback :453-541; reclamation :543-565.
//
// Written here as validate-then-apply: every check of a removal, shift or commit runs over all layers before any
// state changes, so a rejected call leaves the sequence as it was (the reference mutates layer by layer and can
// leave earlier layers changed when a later one throws).
#include <algorithm>
#include <cstdint>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "chromofold/multisequence_cache.h"

namespace {

struct Page {
  uint64_t id = 0;
  uint64_t resident_bytes = 0;
  uint32_t refcount = 0;
  bool retired = false;
};

struct Ref {
  uint64_t page_id = 0;
  uint32_t begin = 0;  // logical token position
  uint32_t count = 0;
};

struct Layer {
  std::vector<Ref> pages;
  uint32_t active_begin = 0, active_count = 0;
  uint64_t active_generation = 0, descriptor_generation = 0;
};

struct Speculation {
  cf_speculation_id id = 0;
  uint32_t baseline = 0;
  uint64_t baseline_generation = 0;
  bool active = false;
};

struct Sequence {
  int64_t id = 0;
  std::vector<Layer> layers;
  uint64_t topology_generation = 0;
  int64_t logical_shift = 0;
  Speculation spec;
};

struct Retired {
  uint64_t page_id = 0, bytes = 0, generation = 0;
};

struct Unsupported : std::runtime_error {
  using std::runtime_error::runtime_error;
};

uint64_t end_of(uint64_t begin, uint64_t count) { return begin + count; }

}  // namespace

struct cf_multisequence_cache {
  cf_multisequence_config config{};
  mutable std::mutex mutex;
  std::map<int64_t, Sequence> sequences;
  std::unordered_map<uint64_t, Page> pages;
  std::vector<Retired> retired;
  cf_multisequence_counters counters{};
  uint64_t generation = 1;
  cf_speculation_id next_speculation = 1;
  std::string error;

  void track_active() {
    counters.active_sequences = sequences.size();
    counters.active_sequences_peak = std::max(counters.active_sequences_peak, counters.active_sequences);
  }

  Page &page(uint64_t id) {
    auto it = pages.find(id);
    if (it == pages.end()) throw std::runtime_error("sequence references an unknown page");
    return it->second;
  }

  void acquire(uint64_t id) {
    Page &p = page(id);
    if (p.retired) throw std::runtime_error("cannot acquire a retired page");
    if (p.refcount == std::numeric_limits<uint32_t>::max()) throw std::runtime_error("page reference count overflow");
    ++p.refcount;
    ++counters.page_ref_increments;
    ++counters.shared_page_references;
    if (p.refcount == 2) ++counters.shared_pages;
  }

  void release(uint64_t id) {
    Page &p = page(id);
    if (p.refcount == 0) throw std::runtime_error("page reference count underflow");
    if (p.refcount == 2 && counters.shared_pages) --counters.shared_pages;
    --p.refcount;
    ++counters.page_ref_decrements;
    if (counters.shared_page_references) --counters.shared_page_references;
    if (p.refcount == 0) {
      p.retired = true;
      retired.push_back({p.id, p.resident_bytes, generation});
      counters.pages_pending_reclamation = retired.size();
      counters.pending_reclamation_bytes += p.resident_bytes;
      counters.pending_reclamation_bytes_peak =
          std::max(counters.pending_reclamation_bytes_peak, counters.pending_reclamation_bytes);
    }
  }

  void release_all(const Sequence &s) {
    for (const Layer &l : s.layers)
      for (const Ref &r : l.pages) release(r.page_id);
  }

  static void check_order(const Layer &l) {
    uint64_t end = 0;
    bool first = true;
    for (const Ref &r : l.pages) {
      if (r.count == 0) throw std::runtime_error("zero-length sealed page reference");
      if (!first && r.begin < end) throw std::runtime_error("overlapping sequence page ranges");
      end = end_of(r.begin, r.count);
      first = false;
    }
    if (!first && l.active_count && l.active_begin < end) throw std::runtime_error("active tail overlaps sealed history");
  }

  bool audit_ok() const {
    try {
      std::unordered_map<uint64_t, uint64_t> seen;
      for (const auto &[id, s] : sequences) {
        if (id != s.id || s.layers.size() != config.layer_count) return false;
        for (const Layer &l : s.layers) {
          check_order(l);
          for (const Ref &r : l.pages) {
            auto p = pages.find(r.page_id);
            if (p == pages.end() || p->second.retired) return false;
            ++seen[r.page_id];
          }
        }
      }
      for (const auto &[id, p] : pages) {
        auto o = seen.find(id);
        const uint64_t n = o == seen.end() ? 0 : o->second;
        if (!p.retired && p.refcount != n) return false;
        if (p.retired && (p.refcount != 0 || n != 0)) return false;
      }
      return true;
    } catch (...) {
      return false;
    }
  }

  void maybe_audit() {
    if (!config.enable_invariant_auditor) return;
    ++counters.invariant_audits;
    if (!audit_ok()) {
      ++counters.invariant_failures;
      throw std::runtime_error("multisequence invariant audit failed");
    }
  }

  Sequence &find(int64_t id) {
    auto it = sequences.find(id);
    if (it == sequences.end()) throw std::runtime_error("sequence does not exist");
    return it->second;
  }

  template <typename Fn>
  int run(Fn &&fn) {
    try {
      fn();
      error.clear();
      return 0;
    } catch (const Unsupported &e) {
      ++counters.unsupported_operations;
      error = e.what();
      return -1;
    } catch (const std::exception &e) {
      error = e.what();
      return -1;
    }
  }
};

extern "C" cf_multisequence_cache *cf_multisequence_create(const cf_multisequence_config *config) {
  if (!config || !config->layer_count || !config->kv_head_count || !config->query_head_count || !config->head_dim ||
      !config->page_size || !config->gqa_group_size ||
      config->query_head_count != config->kv_head_count * config->gqa_group_size)
    return nullptr;
  try {
    auto c = std::make_unique<cf_multisequence_cache>();
    c->config = *config;
    return c.release();
  } catch (...) {
    return nullptr;
  }
}

extern "C" void cf_multisequence_destroy(cf_multisequence_cache *c, void *) { delete c; }

extern "C" int cf_sequence_create(cf_multisequence_cache *c, int64_t id) {
  if (!c) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    if (c->sequences.count(id)) throw std::runtime_error("sequence already exists");
    Sequence s;
    s.id = id;
    s.layers.resize(c->config.layer_count);
    s.topology_generation = ++c->generation;
    c->sequences.emplace(id, std::move(s));
    ++c->counters.sequences_created;
    c->track_active();
    c->maybe_audit();
  });
}

extern "C" int cf_sequence_copy_async(cf_multisequence_cache *c, int64_t src, int64_t dst, uint32_t begin,
                                      uint32_t end, void *) {
  if (!c || src == dst || end < begin) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    auto sit = c->sequences.find(src);
    if (sit == c->sequences.end()) throw std::runtime_error("source sequence does not exist");
    Sequence cand;
    cand.id = dst;
    cand.layers.resize(c->config.layer_count);
    cand.topology_generation = c->generation + 1;
    std::vector<uint64_t> taken;
    try {
      for (uint32_t li = 0; li < c->config.layer_count; ++li) {
        const Layer &from = sit->second.layers[li];
        Layer &to = cand.layers[li];
        for (const Ref &r : from.pages) {
          if (r.begin < begin || end_of(r.begin, r.count) > end) continue;
          c->acquire(r.page_id);
          taken.push_back(r.page_id);
          to.pages.push_back(r);
        }
        if (from.active_count && from.active_begin >= begin && end_of(from.active_begin, from.active_count) <= end) {
          to.active_begin = from.active_begin;
          to.active_count = from.active_count;
          to.active_generation = from.active_generation + 1;
        }
        to.descriptor_generation = from.descriptor_generation + 1;
      }
    } catch (...) {
      for (uint64_t id : taken) c->release(id);
      throw;
    }
    auto old = c->sequences.find(dst);
    if (old != c->sequences.end()) {
      c->release_all(old->second);
      c->sequences.erase(old);
    }
    c->sequences.emplace(dst, std::move(cand));
    ++c->generation;
    ++c->counters.sequences_copied;
    c->track_active();
    c->maybe_audit();
  });
}

extern "C" int cf_sequence_remove_async(cf_multisequence_cache *c, int64_t id, int64_t pb, int64_t pe, void *) {
  if (!c || pe < pb) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    Sequence &s = c->find(id);
    if (pb < 0 && pe < 0) {
      c->release_all(s);
      c->sequences.erase(id);
      ++c->counters.sequences_removed;
      ++c->generation;
      c->track_active();
      c->maybe_audit();
      return;
    }
    if (pb < 0) pb = 0;
    // validate every layer first
    std::vector<uint32_t> new_active(s.layers.size());
    for (size_t li = 0; li < s.layers.size(); ++li) {
      const Layer &l = s.layers[li];
      for (const Ref &r : l.pages) {
        const int64_t rb = r.begin, re = rb + r.count;
        if (re <= pb || rb >= pe) continue;
        if (pb > rb || pe < re) throw Unsupported("removal inside immutable page is not supported");
      }
      const int64_t ab = l.active_begin, ae = ab + l.active_count;
      if (pb <= ab && pe >= ae) new_active[li] = 0;
      else if (pb >= ab && pb < ae && pe >= ae) new_active[li] = static_cast<uint32_t>(pb - ab);
      else if (pe > ab && pb < ae) throw Unsupported("non-suffix active-tail removal is not supported");
      else new_active[li] = l.active_count;
    }
    for (size_t li = 0; li < s.layers.size(); ++li) {
      Layer &l = s.layers[li];
      std::vector<Ref> kept;
      kept.reserve(l.pages.size());
      for (const Ref &r : l.pages) {
        const int64_t rb = r.begin, re = rb + r.count;
        if (re <= pb || rb >= pe) kept.push_back(r);
        else c->release(r.page_id);
      }
      l.pages = std::move(kept);
      l.active_count = new_active[li];
      ++l.descriptor_generation;
    }
    ++s.topology_generation;
    ++c->generation;
    ++c->counters.sequences_removed;
    c->maybe_audit();
  });
}

extern "C" int cf_sequence_shift_async(cf_multisequence_cache *c, int64_t id, uint32_t pb, uint32_t pe, int32_t delta,
                                       void *) {
  if (!c || pe < pb) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    Sequence &s = c->find(id);
    std::vector<Layer> next = s.layers;  // shift a copy, then commit it
    for (Layer &l : next) {
      for (Ref &r : l.pages) {
        const uint64_t re = end_of(r.begin, r.count);
        if (r.begin >= pb && re <= pe) {
          const int64_t moved = int64_t(r.begin) + delta;
          if (moved < 0) throw std::runtime_error("context shift produces negative token position");
          r.begin = static_cast<uint32_t>(moved);
        } else if (r.begin < pe && re > pb) {
          throw Unsupported("context shift must align with immutable page boundaries");
        }
      }
      if (l.active_count && l.active_begin >= pb && end_of(l.active_begin, l.active_count) <= pe) {
        const int64_t moved = int64_t(l.active_begin) + delta;
        if (moved < 0) throw std::runtime_error("context shift produces negative active position");
        l.active_begin = static_cast<uint32_t>(moved);
      }
      cf_multisequence_cache::check_order(l);
      ++l.descriptor_generation;
    }
    s.layers = std::move(next);
    s.logical_shift += delta;
    ++s.topology_generation;
    ++c->generation;
    ++c->counters.sequences_shifted;
    c->maybe_audit();
  });
}

extern "C" int cf_sequence_append_async(cf_multisequence_cache *c, int64_t id, uint32_t layer, uint32_t token_begin,
                                        const cf_device_tensor_view *keys, const cf_device_tensor_view *values,
                                        void *) {
  if (!c || !keys || !values || layer >= c->config.layer_count || cf_device_tensor_validate(keys) != 0 ||
      cf_device_tensor_validate(values) != 0)
    return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    Sequence &s = c->find(id);
    if (keys->token_count != values->token_count || keys->head_count != values->head_count ||
        keys->head_dim != values->head_dim || keys->head_count != c->config.kv_head_count ||
        keys->head_dim != c->config.head_dim)
      throw std::runtime_error("append tensor topology mismatch");
    Layer &l = s.layers[layer];
    if (l.active_count && token_begin != l.active_begin + l.active_count)
      throw std::runtime_error("non-contiguous sequence append");
    if (uint64_t(l.active_count) + keys->token_count > c->config.page_size)
      throw std::runtime_error("append crosses sequence active-page boundary");
    if (!l.active_count) l.active_begin = token_begin;
    l.active_count += keys->token_count;
    ++l.active_generation;
    ++s.topology_generation;
    ++c->generation;
    c->maybe_audit();
  });
}

extern "C" int cf_multisequence_attention_async(cf_multisequence_cache *c, const cf_sequence_attention_item *items,
                                                uint32_t n, void *) {
  if (!c || !items || n == 0) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    std::set<int64_t> seqs;
    for (uint32_t i = 0; i < n; ++i) {
      if (!c->sequences.count(items[i].sequence_id))
        throw std::runtime_error("attention item references unknown sequence");
      if (items[i].layer >= c->config.layer_count || cf_device_tensor_validate(&items[i].query) != 0 ||
          !items[i].output)
        throw std::runtime_error("invalid sequence attention item");
      seqs.insert(items[i].sequence_id);
    }
    ++c->counters.batches_dispatched;
    c->counters.sequences_per_batch_peak = std::max<uint64_t>(c->counters.sequences_per_batch_peak, seqs.size());
    throw Unsupported("the multi-sequence cache holds no KV data: attention over shared pages runs through "
                      "cf_ms_cuda_execute_batch_async; dense fallback is forbidden");
  });
}

extern "C" cf_speculation_id cf_sequence_speculation_begin(cf_multisequence_cache *c, int64_t id) {
  if (!c) return 0;
  std::lock_guard<std::mutex> g(c->mutex);
  cf_speculation_id out = 0;
  c->run([&] {
    Sequence &s = c->find(id);
    if (s.spec.active) throw std::runtime_error("speculation already active");
    uint32_t baseline = 0;
    for (const Layer &l : s.layers) baseline = std::max(baseline, l.active_count);
    out = c->next_speculation++;
    s.spec = {out, baseline, s.topology_generation, true};
    ++c->counters.speculative_transactions_started;
  });
  return out;
}

extern "C" int cf_sequence_speculation_commit(cf_multisequence_cache *c, int64_t id, cf_speculation_id spec,
                                              uint32_t accepted, void *) {
  if (!c || spec == 0) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    auto it = c->sequences.find(id);
    if (it == c->sequences.end() || !it->second.spec.active || it->second.spec.id != spec)
      throw std::runtime_error("invalid speculative transaction");
    Sequence &s = it->second;
    const uint32_t base = s.spec.baseline;
    for (const Layer &l : s.layers) {
      if (l.active_count < base) throw std::runtime_error("active tail predates speculative baseline");
      if (accepted > l.active_count - base) throw std::runtime_error("accepted token count exceeds provisional tail");
    }
    for (Layer &l : s.layers) {
      l.active_count = base + accepted;
      ++l.active_generation;
    }
    s.spec = {};
    ++s.topology_generation;
    ++c->generation;
    ++c->counters.speculative_transactions_committed;
    c->maybe_audit();
  });
}

extern "C" int cf_sequence_speculation_rollback(cf_multisequence_cache *c, int64_t id, cf_speculation_id spec, void *) {
  if (!c || spec == 0) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    auto it = c->sequences.find(id);
    if (it == c->sequences.end() || !it->second.spec.active || it->second.spec.id != spec)
      throw std::runtime_error("invalid speculative transaction");
    Sequence &s = it->second;
    for (Layer &l : s.layers) {
      l.active_count = s.spec.baseline;
      ++l.active_generation;
    }
    s.topology_generation = s.spec.baseline_generation;
    s.spec = {};
    ++c->generation;
    ++c->counters.speculative_transactions_rolled_back;
    c->maybe_audit();
  });
}

extern "C" int cf_multisequence_reclaim_async(cf_multisequence_cache *c, void *) {
  if (!c) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->run([&] {
    for (const Retired &r : c->retired) {
      auto p = c->pages.find(r.page_id);
      if (p == c->pages.end() || p->second.refcount != 0) throw std::runtime_error("invalid page in reclamation queue");
    }
    for (const Retired &r : c->retired) {
      c->pages.erase(r.page_id);
      ++c->counters.pages_reclaimed;
      c->counters.pending_reclamation_bytes -= r.bytes;
    }
    c->retired.clear();
    c->counters.pages_pending_reclamation = 0;
    c->maybe_audit();
  });
}

extern "C" int cf_multisequence_audit(const cf_multisequence_cache *c) {
  if (!c) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  return c->audit_ok() ? 0 : -1;
}

extern "C" int cf_multisequence_get_counters(const cf_multisequence_cache *c, cf_multisequence_counters *out) {
  if (!c || !out) return -1;
  std::lock_guard<std::mutex> g(c->mutex);
  *out = c->counters;
  return 0;
}

extern "C" const char *cf_multisequence_last_error(const cf_multisequence_cache *c) {
  return c ? c->error.c_str() : "null multisequence cache";
}
