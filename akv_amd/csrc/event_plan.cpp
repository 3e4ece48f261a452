// Host event compiler: Drop / Reposition replay over the raw token stream.
//
// Same results and error messages as the reference's CPU compiler,
// count_radix_reposition_transitions + compile_radix_reposition_layout
// (akv/system/sglang/kernels/ops/attention/context_plan.py:80-532), behind a
// plain C ABI instead of tvm-ffi.  One replay routine drives both entry
// points through a sink (counting vs filling), so the count and fill passes
// cannot disagree.
//
// Replay: active raw tokens form a doubly linked list.  A Drop at insertion
// i unlinks the still-kept tokens of its ordered, disjoint ranges and marks
// the first surviving successor as "unsettled" (its position no longer equals
// its rank).  A Reposition at insertion i renumbers the active suffix from the
// first unsettled token, continuing after its predecessor's position, and
// emits one (raw, old, new) transition per token.  A token is born at
// next_position++.  Drop precedes Reposition at a shared insertion point.
#include <cstdint>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "abi_common.h"

namespace akv {
namespace {

constexpr int32_t kTokenRecord = 0;
constexpr int32_t kDeltaRecord = 1;
constexpr int32_t kRepositionRecord = 2;

struct Program {
  int64_t n;
  const int32_t* drops;
  int64_t drop_count;
  const int32_t* drop_offsets;
  const int32_t* ranges;
  int64_t range_count;
  const int32_t* boundaries;
  const int32_t* inserts;
  int64_t repo_count;
};

void require(bool ok, const char* message) {
  if (!ok) throw std::invalid_argument(message);
}

// Metadata checks, in the order the reference's count pass makes them.
void validate(const Program& p, int64_t ranges_len) {
  require(p.n >= 0 && p.n <= std::numeric_limits<int32_t>::max(),
          "token_count exceeds the int32 Reposition limit");
  require(ranges_len % 2 == 0, "Reposition transition-count tensor lengths are inconsistent");
  require(p.drop_offsets[0] == 0 && p.drop_offsets[p.drop_count] == p.range_count,
          "drop_range_offsets does not cover drop_ranges");
  for (int64_t i = 0; i < p.drop_count; ++i)
    require(p.drops[i] >= 0 && p.drops[i] <= p.n && (i == 0 || p.drops[i - 1] < p.drops[i]) &&
                p.drop_offsets[i] < p.drop_offsets[i + 1],
            "Invalid Drop event metadata");
  for (int64_t i = 0; i < p.repo_count; ++i)
    require(p.inserts[i] == p.boundaries[i] + 1 && p.inserts[i] > 0 && p.inserts[i] <= p.n &&
                (i == 0 || p.boundaries[i - 1] < p.boundaries[i]),
            "Invalid Reposition event metadata");
}

// Receives the replay's events.  The counting sink only counts transitions.
struct Sink {
  virtual ~Sink() = default;
  virtual void birth(int32_t token, int32_t position, int32_t stage) = 0;
  virtual void reposition(int64_t index, bool effective, int32_t stage) = 0;
  virtual void transition(int64_t index, int32_t token, int32_t old_position, int32_t new_position,
                          int32_t stage) = 0;
  virtual void stage_end(int32_t stage, int64_t cursor) = 0;
};

struct ReplayResult {
  int status = 0;  // 0 ok, 1 reposition with no active token
  int32_t bad_boundary = -1;
  int32_t stages = 0;
  int32_t next_position = 0;
  std::vector<int32_t> position;
  std::vector<uint8_t> kept;
};

ReplayResult replay(const Program& p, Sink& sink) {
  const int32_t n = static_cast<int32_t>(p.n);
  ReplayResult out;
  out.position.assign(n, -1);
  out.kept.assign(n, 0);
  std::vector<int32_t> prev(n, -1), next(n, -1);
  int32_t* pos = out.position.data();
  uint8_t* kept = out.kept.data();
  int32_t tail = -1, unsettled = -1, active = 0, next_position = 0, stage = 0;
  int64_t d = 0, r = 0, cursor = 0;
  for (int32_t at = 0; at <= n; ++at) {
    if (d < p.drop_count && p.drops[d] == at) {
      int32_t last_end = -1;
      for (int32_t q = p.drop_offsets[d]; q < p.drop_offsets[d + 1]; ++q) {
        const int32_t start = p.ranges[2 * q], end = p.ranges[2 * q + 1];
        require(start >= 0 && start < end && end <= at && (q == p.drop_offsets[d] || last_end < start),
                "Drop ranges must be ordered, disjoint, and already materialized");
        last_end = end;
        for (int32_t t = start; t < end; ++t) {
          if (!kept[t]) continue;
          const int32_t before = prev[t], after = next[t];
          if (before >= 0) next[before] = after;
          if (after >= 0)
            prev[after] = before;
          else
            tail = before;
          kept[t] = 0;
          --active;
          if (unsettled == t) unsettled = after;
          if (after >= 0 && (unsettled < 0 || after < unsettled)) unsettled = after;
        }
      }
      if (active == 0) unsettled = -1;
      ++d;
    }
    if (r < p.repo_count && p.inserts[r] == at) {
      if (active == 0) {
        out.status = 1;
        out.bad_boundary = p.boundaries[r];
        return out;
      }
      if (unsettled < 0) {
        sink.reposition(r, false, -1);
      } else {
        ++stage;
        sink.reposition(r, true, stage);
        int32_t rank = prev[unsettled] < 0 ? 0 : pos[prev[unsettled]] + 1;
        for (int32_t t = unsettled; t >= 0; t = next[t]) {
          require(pos[t] > rank, "Non-compact active suffix invariant was violated");
          sink.transition(cursor++, t, pos[t], rank, stage);
          pos[t] = rank++;
        }
        next_position = active;
        unsettled = -1;
        sink.stage_end(stage, cursor);
      }
      ++r;
    }
    if (at == n) continue;
    const int32_t rank = active;
    kept[at] = 1;
    pos[at] = next_position++;
    sink.birth(at, pos[at], stage);
    prev[at] = tail;
    if (tail >= 0) next[tail] = at;
    tail = at;
    ++active;
    if (unsettled < 0 && pos[at] != rank) unsettled = at;
  }
  out.stages = stage;
  out.next_position = next_position;
  return out;
}

struct CountSink final : Sink {
  int32_t* per_reposition;
  int64_t current = -1;
  explicit CountSink(int32_t* counts) : per_reposition(counts) {}
  void birth(int32_t, int32_t, int32_t) override {}
  void reposition(int64_t index, bool, int32_t) override { current = index; }
  void transition(int64_t, int32_t, int32_t, int32_t, int32_t) override { ++per_reposition[current]; }
  void stage_end(int32_t, int64_t) override {}
};

struct FillSink final : Sink {
  int32_t* materialized_stage;
  int32_t* birth_positions;
  int32_t* birth_stages;
  int32_t* transition_offsets;
  int32_t* raw;
  int32_t* old_pos;
  int32_t* new_pos;
  int64_t capacity;
  int32_t* effective_stage;
  uint8_t* effective;
  uint8_t* ignored;
  void birth(int32_t token, int32_t position, int32_t stage) override {
    birth_positions[token] = position;
    birth_stages[token] = stage;
    materialized_stage[token] = stage;
  }
  void reposition(int64_t index, bool eff, int32_t stage) override {
    effective[index] = eff ? 1 : 0;
    ignored[index] = eff ? 0 : 1;
    effective_stage[index] = eff ? stage : -1;
  }
  void transition(int64_t index, int32_t token, int32_t o, int32_t nw, int32_t stage) override {
    require(index < capacity, "Reposition transition output capacity is too small");
    raw[index] = token;
    old_pos[index] = o;
    new_pos[index] = nw;
    materialized_stage[token] = stage;
  }
  void stage_end(int32_t stage, int64_t cursor) override {
    transition_offsets[stage] = static_cast<int32_t>(cursor);
  }
};

Program make_program(int64_t token_count, const int32_t* drops, int64_t drop_count,
                     const int32_t* drop_offsets, const int32_t* ranges, int64_t ranges_len,
                     const int32_t* boundaries, const int32_t* inserts, int64_t repo_count) {
  Program p{};
  p.n = token_count;
  p.drops = drops;
  p.drop_count = drop_count;
  p.drop_offsets = drop_offsets;
  p.ranges = ranges;
  p.range_count = ranges_len / 2;
  p.boundaries = boundaries;
  p.inserts = inserts;
  p.repo_count = repo_count;
  return p;
}

}  // namespace
}  // namespace akv

extern "C" int akv_plan_count(int64_t token_count, const int32_t* drop_insert_offsets, int64_t drop_count,
                              const int32_t* drop_range_offsets, const int32_t* drop_ranges,
                              int64_t drop_ranges_len, const int32_t* reposition_raw_boundaries,
                              const int32_t* reposition_insert_offsets, int64_t reposition_count,
                              int32_t* transition_counts, int64_t* status) {
  using namespace akv;
  if (drop_count < 0 || drop_ranges_len < 0 || reposition_count < 0 || !drop_range_offsets || !status ||
      (reposition_count > 0 && !transition_counts))
    return fail(AKV_EINVAL, "Reposition transition-count tensor lengths are inconsistent");
  try {
    const Program p = make_program(token_count, drop_insert_offsets, drop_count, drop_range_offsets,
                                   drop_ranges, drop_ranges_len, reposition_raw_boundaries,
                                   reposition_insert_offsets, reposition_count);
    validate(p, drop_ranges_len);
    for (int64_t i = 0; i < reposition_count; ++i) transition_counts[i] = 0;
    CountSink sink(transition_counts);
    const ReplayResult res = replay(p, sink);
    status[0] = res.status;
    status[1] = res.status ? res.bad_boundary : -1;
  } catch (const std::exception& e) {
    return fail(AKV_EINVAL, "%s", e.what());
  }
  return AKV_OK;
}

extern "C" int akv_plan_compile(const void* token_ids, int32_t token_ids_dtype, int64_t token_count,
                                const int32_t* drop_insert_offsets, int64_t drop_count,
                                const int32_t* drop_range_offsets, const int32_t* drop_ranges,
                                int64_t drop_ranges_len, const int32_t* reposition_raw_boundaries,
                                const int32_t* reposition_insert_offsets, int64_t reposition_count,
                                int32_t* records, uint8_t* virtual_mask, int64_t* key_to_token,
                                int64_t record_capacity, int64_t* token_to_key, int32_t* positions,
                                uint8_t* keep_mask, int32_t* materialized_stage, int32_t* birth_positions,
                                int32_t* birth_stages, int32_t* transition_offsets,
                                int32_t* transition_raw_tokens, int32_t* transition_old_positions,
                                int32_t* transition_new_positions, int64_t transition_capacity,
                                int32_t* effective_reposition_stages, int64_t* drop_event_to_key,
                                uint8_t* effective_repositions, uint8_t* ignored_repositions,
                                int64_t* status) {
  using namespace akv;
  if (token_ids_dtype != AKV_I32 && token_ids_dtype != AKV_I64)
    return fail(AKV_EINVAL, "token_ids must be a CPU int32/int64 vector");
  if (drop_count < 0 || drop_ranges_len < 0 || reposition_count < 0 || !drop_range_offsets || !status)
    return fail(AKV_EINVAL, "Reposition output lengths are inconsistent");
  if (record_capacity < token_count + drop_ranges_len / 2 + reposition_count)
    return fail(AKV_EINVAL, "Radix output capacity is too small");
  try {
    const Program p = make_program(token_count, drop_insert_offsets, drop_count, drop_range_offsets,
                                   drop_ranges, drop_ranges_len, reposition_raw_boundaries,
                                   reposition_insert_offsets, reposition_count);
    validate(p, drop_ranges_len);
    for (int64_t i = 0; i < reposition_count; ++i) {
      effective_repositions[i] = 0;
      ignored_repositions[i] = 0;
      effective_reposition_stages[i] = -1;
    }
    transition_offsets[0] = 0;
    FillSink sink;
    sink.materialized_stage = materialized_stage;
    sink.birth_positions = birth_positions;
    sink.birth_stages = birth_stages;
    sink.transition_offsets = transition_offsets;
    sink.raw = transition_raw_tokens;
    sink.old_pos = transition_old_positions;
    sink.new_pos = transition_new_positions;
    sink.capacity = transition_capacity;
    sink.effective_stage = effective_reposition_stages;
    sink.effective = effective_repositions;
    sink.ignored = ignored_repositions;
    const ReplayResult res = replay(p, sink);
    if (res.status) {
      status[0] = 1;
      status[4] = res.bad_boundary;
      return AKV_OK;
    }
    const int32_t n = static_cast<int32_t>(token_count);
    for (int32_t t = 0; t < n; ++t) {
      positions[t] = res.position[t];
      keep_mask[t] = res.kept[t];
    }
    int64_t transitions = res.stages ? transition_offsets[res.stages] : 0;
    require(transitions == transition_capacity, "Reposition transition count/fill passes disagree");

    // Radix key records: one per Drop range, per effective Reposition and per token.
    const int32_t* ids32 = token_ids_dtype == AKV_I32 ? static_cast<const int32_t*>(token_ids) : nullptr;
    const int64_t* ids64 = token_ids_dtype == AKV_I64 ? static_cast<const int64_t*>(token_ids) : nullptr;
    int64_t key = 0, d = 0, r = 0;
    auto emit = [&](int32_t kind, int32_t a, int32_t b, bool is_virtual, int64_t token) {
      records[3 * key] = kind;
      records[3 * key + 1] = a;
      records[3 * key + 2] = b;
      virtual_mask[key] = is_virtual ? 1 : 0;
      key_to_token[key] = token;
      ++key;
    };
    for (int32_t at = 0; at <= n; ++at) {
      if (d < drop_count && drop_insert_offsets[d] == at) {
        drop_event_to_key[d] = key;
        for (int32_t q = drop_range_offsets[d]; q < drop_range_offsets[d + 1]; ++q)
          emit(kDeltaRecord, static_cast<int32_t>(-static_cast<int64_t>(drop_ranges[2 * q]) - 1),
               static_cast<int32_t>(-static_cast<int64_t>(drop_ranges[2 * q + 1]) - 1), true, -1);
        ++d;
      }
      if (r < reposition_count && reposition_insert_offsets[r] == at) {
        if (effective_repositions[r]) emit(kRepositionRecord, reposition_raw_boundaries[r], -1, true, -1);
        ++r;
      }
      if (at == n) continue;
      token_to_key[at] = key;
      const int64_t id = ids32 ? ids32[at] : ids64[at];
      if (id < 0 || id > std::numeric_limits<int32_t>::max()) {
        status[0] = 2;
        status[4] = id;
        return AKV_OK;
      }
      emit(kTokenRecord, static_cast<int32_t>(id), res.position[at], false, at);
    }
    status[0] = 0;
    status[1] = key;
    status[2] = res.stages;
    status[3] = res.next_position;
    status[4] = -1;
  } catch (const std::exception& e) {
    return fail(AKV_EINVAL, "%s", e.what());
  }
  return AKV_OK;
}
