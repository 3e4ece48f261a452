// Host occurrence-window compiler: which (raw token, position) versions a
// forward's attention reads and in which order they are first needed.
//
// Same results and error messages as compile_occurrence_window
// (akv/system/sglang/srt/context_system/occurrence.py:112-265), in C++ behind
// the C ABI.  One replay routine drives the count and the fill entry points
// through a sink, so both passes agree; the fill checks every write against
// the caller's counts.
//
// Replay: every raw token starts as its birth occurrence (id = raw index) at
// its birth position.  Stages are walked in order; a stage first applies its
// Reposition transitions to the current positions, then its queries are
// split into segments at the visibility expiries that fall inside them.  A
// segment [start, end) reads every earlier token still visible at start
// (visible_until > start) at its current position -- a token whose current
// position differs from its last materialised one gets a new occurrence id
// -- followed by its own birth occurrences.  After the last stage every raw
// token is materialised at its terminal position.
#include <algorithm>
#include <cstdint>
#include <limits>
#include <stdexcept>
#include <vector>

#include "abi_common.h"

namespace akv {
namespace {

struct Inputs {
  int64_t n;
  const int32_t* birth;
  const int32_t* stages;
  const int32_t* offsets;
  int64_t stage_count;
  const int32_t* changed;
  const int32_t* old_pos;
  const int32_t* new_pos;
  const int32_t* expiry;
  const int32_t* terminal;
  int64_t query_start, query_end;
};

void require(bool ok, const char* message) {
  if (!ok) throw std::invalid_argument(message);
}

void fail_runtime(const char* message) { throw std::runtime_error(message); }

// Output sink: counts, or fills caller arrays of the counted sizes, or
// (bounded) fills what fits in the caller's capacities and counts the rest.
struct Sink {
  bool fill = false;
  bool bounded = false;
  int64_t occurrences = 0, segments = 0, keys = 0, first_final = 0;
  int32_t* occ_raw = nullptr;
  int32_t* occ_pos = nullptr;
  int32_t* terminal_occ = nullptr;
  int32_t* seg_start = nullptr;
  int32_t* seg_end = nullptr;
  int32_t* key_offsets = nullptr;
  int32_t* key_occ = nullptr;

  // fill mode: capacities of the caller's arrays; every write is checked
  int64_t cap_occurrences = 0, cap_segments = 0, cap_keys = 0;
  static void overflow() {
    throw std::invalid_argument("akv_window_compile: output capacities do not match the window");
  }
  void occurrence(int32_t raw, int32_t pos) {
    if (fill) {
      if (occurrences < cap_occurrences) {
        occ_raw[occurrences] = raw;
        occ_pos[occurrences] = pos;
      } else if (!bounded) {
        overflow();
      }
    }
    ++occurrences;
  }
  void key(int32_t id) {
    if (fill) {
      if (keys < cap_keys)
        key_occ[keys] = id;
      else if (!bounded)
        overflow();
    }
    ++keys;
  }
  void segment(int32_t start, int32_t end) {
    if (fill) {
      if (segments < cap_segments) {
        seg_start[segments] = start;
        seg_end[segments] = end;
        key_offsets[segments + 1] = static_cast<int32_t>(keys);
      } else if (!bounded) {
        overflow();
      }
    }
    ++segments;
  }
};

void validate(const Inputs& in) {
  const int64_t n = in.n;
  require(n >= 1, "Compact occurrence birth metadata must cover a nonempty prompt.");
  require(0 <= in.query_start && in.query_start < in.query_end && in.query_end <= n,
          "Occurrence query window is outside the raw prompt.");
  require(in.stage_count >= 0, "Occurrence transition offsets require an initial zero.");
  require(in.offsets[0] == 0, "Occurrence transition offsets must start at zero and be monotonic.");
  for (int64_t s = 0; s < in.stage_count; ++s)
    require(in.offsets[s + 1] >= in.offsets[s], "Occurrence transition offsets must start at zero and be monotonic.");
  for (int64_t i = 0; i < n; ++i) require(in.birth[i] >= 0, "Occurrence positions must be non-negative.");
  const int64_t total = in.offsets[in.stage_count];
  for (int64_t i = 0; i < total; ++i) require(in.new_pos[i] >= 0, "Occurrence positions must be non-negative.");
  for (int64_t i = 0; i < n; ++i)
    require(in.stages[i] >= 0 && in.stages[i] <= in.stage_count,
            "Occurrence birth stages are outside the Reposition program.");
  for (int64_t i = 1; i < n; ++i)
    require(in.stages[i] >= in.stages[i - 1], "Occurrence birth stages must preserve raw-token order.");
  for (int64_t i = 0; i < n; ++i)
    require(in.expiry[i] > i, "A token cannot become invisible before it has been computed.");
}

void replay(const Inputs& in, Sink& out) {
  validate(in);
  const int64_t n = in.n;
  const int64_t S = in.stage_count;
  // bounds[s] = first raw token born at stage >= s
  std::vector<int64_t> bounds(S + 2);
  for (int64_t s = 0; s <= S + 1; ++s)
    bounds[s] = std::lower_bound(in.stages, in.stages + n, static_cast<int32_t>(s)) - in.stages;
  std::vector<int32_t> cur_id(n), cur_pos(n), mat_pos(n);
  for (int64_t i = 0; i < n; ++i) {
    cur_id[i] = static_cast<int32_t>(i);
    cur_pos[i] = mat_pos[i] = in.birth[i];
    out.occurrence(static_cast<int32_t>(i), in.birth[i]);
  }
  auto materialize = [&](int64_t u) {
    if (mat_pos[u] == cur_pos[u]) return;
    if (out.occurrences + 1 > std::numeric_limits<int32_t>::max())
      throw std::invalid_argument("Occurrence IDs exceed int32 capacity.");
    cur_id[u] = static_cast<int32_t>(out.occurrences);
    mat_pos[u] = cur_pos[u];
    out.occurrence(static_cast<int32_t>(u), cur_pos[u]);
  };
  std::vector<int32_t> cuts;
  std::vector<uint8_t> seen(n, 0);
  int64_t covered = in.query_start;
  for (int64_t stage = 0; stage <= S; ++stage) {
    if (stage) {
      const int64_t b = in.offsets[stage - 1], e = in.offsets[stage];
      for (int64_t i = b; i < e; ++i)
        require(in.changed[i] >= 0 && in.changed[i] < n, "Reposition transition references an invalid raw token.");
      for (int64_t i = b; i < e; ++i) {
        require(!seen[in.changed[i]], "One Reposition stage cannot transition a raw token twice.");
        seen[in.changed[i]] = 1;
      }
      for (int64_t i = b; i < e; ++i) seen[in.changed[i]] = 0;
      for (int64_t i = b; i < e; ++i)
        require(cur_pos[in.changed[i]] == in.old_pos[i],
                "Reposition transition old positions do not match current state.");
      for (int64_t i = b; i < e; ++i) cur_pos[in.changed[i]] = in.new_pos[i];
    }
    const int64_t ls = std::max(in.query_start, bounds[stage]);
    const int64_t le = std::min(in.query_end, bounds[stage + 1]);
    if (ls >= le) continue;
    if (ls != covered) fail_runtime("Occurrence stages do not cover the requested query window.");
    cuts.clear();
    cuts.push_back(static_cast<int32_t>(ls));
    for (int64_t u = 0; u < le; ++u)
      if (in.expiry[u] > ls && in.expiry[u] < le) cuts.push_back(in.expiry[u]);
    std::sort(cuts.begin() + 1, cuts.end());
    cuts.erase(std::unique(cuts.begin() + 1, cuts.end()), cuts.end());
    cuts.push_back(static_cast<int32_t>(le));
    for (size_t c = 0; c + 1 < cuts.size(); ++c) {
      const int64_t start = cuts[c], end = cuts[c + 1];
      for (int64_t u = 0; u < start; ++u)
        if (in.expiry[u] > start) materialize(u);
      for (int64_t u = 0; u < start; ++u)
        if (in.expiry[u] > start) out.key(cur_id[u]);
      for (int64_t u = start; u < end; ++u) out.key(static_cast<int32_t>(u));
      out.segment(static_cast<int32_t>(start), static_cast<int32_t>(end));
    }
    covered = le;
  }
  if (covered != in.query_end) fail_runtime("Occurrence stages do not cover the requested query window.");
  for (int64_t i = 0; i < n; ++i)
    require(cur_pos[i] == in.terminal[i], "Compact occurrence transitions disagree with terminal Radix positions.");
  out.first_final = out.occurrences;
  for (int64_t u = 0; u < n; ++u) materialize(u);
  if (out.keys > std::numeric_limits<int32_t>::max())
    throw std::invalid_argument("Occurrence segment offsets exceed int32 capacity.");
  if (out.fill)
    for (int64_t u = 0; u < n; ++u) out.terminal_occ[u] = cur_id[u];
}

int run(const Inputs& in, Sink& sink) {
  try {
    replay(in, sink);
  } catch (const std::invalid_argument& e) {
    return fail(AKV_EINVAL, "%s", e.what());
  } catch (const std::runtime_error& e) {
    return fail(AKV_ERUNTIME, "%s", e.what());
  } catch (const std::bad_alloc&) {
    return fail(AKV_EINVAL, "occurrence window: out of host memory");
  }
  return AKV_OK;
}

bool null_inputs(const int32_t* birth, const int32_t* stages, const int32_t* offsets, const int32_t* expiry,
                 const int32_t* terminal) {
  return !birth || !stages || !offsets || !expiry || !terminal;
}

Sink fill_sink(const int64_t* capacities, int32_t* occ_raw, int32_t* occ_pos, int32_t* terminal_occ,
               int32_t* seg_start, int32_t* seg_end, int32_t* key_offsets, int32_t* key_occ) {
  Sink sink;
  sink.fill = true;
  sink.cap_occurrences = capacities[0];
  sink.cap_segments = capacities[1];
  sink.cap_keys = capacities[2];
  sink.occ_raw = occ_raw;
  sink.occ_pos = occ_pos;
  sink.terminal_occ = terminal_occ;
  sink.seg_start = seg_start;
  sink.seg_end = seg_end;
  sink.key_offsets = key_offsets;
  sink.key_occ = key_occ;
  key_offsets[0] = 0;
  return sink;
}

}  // namespace
}  // namespace akv

extern "C" int akv_window_count(int64_t n, const int32_t* birth_positions, const int32_t* birth_stages,
                                const int32_t* transition_offsets, int64_t stage_count,
                                const int32_t* transition_raw_tokens, const int32_t* transition_old_positions,
                                const int32_t* transition_new_positions, const int32_t* visible_until,
                                const int32_t* terminal_positions, int64_t query_start, int64_t query_end,
                                int64_t* counts) {
  using namespace akv;
  if (!counts || null_inputs(birth_positions, birth_stages, transition_offsets, visible_until, terminal_positions))
    return fail(AKV_EINVAL, "akv_window_count: null host pointer");
  Inputs in{n, birth_positions, birth_stages, transition_offsets, stage_count, transition_raw_tokens,
            transition_old_positions, transition_new_positions, visible_until, terminal_positions,
            query_start, query_end};
  Sink sink;
  const int rc = run(in, sink);
  if (rc) return rc;
  counts[0] = sink.occurrences;
  counts[1] = sink.segments;
  counts[2] = sink.keys;
  counts[3] = sink.first_final;
  return AKV_OK;
}

extern "C" int akv_window_compile(int64_t n, const int32_t* birth_positions, const int32_t* birth_stages,
                                  const int32_t* transition_offsets, int64_t stage_count,
                                  const int32_t* transition_raw_tokens, const int32_t* transition_old_positions,
                                  const int32_t* transition_new_positions, const int32_t* visible_until,
                                  const int32_t* terminal_positions, int64_t query_start, int64_t query_end,
                                  const int64_t* counts, int32_t* occurrence_raw_tokens,
                                  int32_t* occurrence_positions, int32_t* terminal_occurrences,
                                  int32_t* segment_query_starts, int32_t* segment_query_ends,
                                  int32_t* segment_key_offsets, int32_t* segment_key_occurrences) {
  using namespace akv;
  if (!counts || null_inputs(birth_positions, birth_stages, transition_offsets, visible_until, terminal_positions) ||
      !occurrence_raw_tokens || !occurrence_positions || !terminal_occurrences || !segment_query_starts ||
      !segment_query_ends || !segment_key_offsets || !segment_key_occurrences)
    return fail(AKV_EINVAL, "akv_window_compile: null host pointer");
  Inputs in{n, birth_positions, birth_stages, transition_offsets, stage_count, transition_raw_tokens,
            transition_old_positions, transition_new_positions, visible_until, terminal_positions,
            query_start, query_end};
  // one replay: every write is bounded by the caller's counts, and the
  // counts must come out exact
  if (counts[0] < 0 || counts[1] < 0 || counts[2] < 0)
    return fail(AKV_EINVAL, "akv_window_compile: output capacities do not match the window");
  Sink sink = fill_sink(counts, occurrence_raw_tokens, occurrence_positions, terminal_occurrences,
                        segment_query_starts, segment_query_ends, segment_key_offsets, segment_key_occurrences);
  const int rc = run(in, sink);
  if (rc) return rc;
  if (sink.occurrences != counts[0] || sink.segments != counts[1] || sink.keys != counts[2])
    return fail(AKV_EINVAL, "akv_window_compile: output capacities do not match the window");
  return AKV_OK;
}

extern "C" int akv_window_compile_bounded(int64_t n, const int32_t* birth_positions, const int32_t* birth_stages,
                                          const int32_t* transition_offsets, int64_t stage_count,
                                          const int32_t* transition_raw_tokens,
                                          const int32_t* transition_old_positions,
                                          const int32_t* transition_new_positions, const int32_t* visible_until,
                                          const int32_t* terminal_positions, int64_t query_start,
                                          int64_t query_end, const int64_t* capacities, int64_t* counts,
                                          int32_t* occurrence_raw_tokens, int32_t* occurrence_positions,
                                          int32_t* terminal_occurrences, int32_t* segment_query_starts,
                                          int32_t* segment_query_ends, int32_t* segment_key_offsets,
                                          int32_t* segment_key_occurrences) {
  using namespace akv;
  if (!capacities || !counts ||
      null_inputs(birth_positions, birth_stages, transition_offsets, visible_until, terminal_positions) ||
      !occurrence_raw_tokens || !occurrence_positions || !terminal_occurrences || !segment_query_starts ||
      !segment_query_ends || !segment_key_offsets || !segment_key_occurrences)
    return fail(AKV_EINVAL, "akv_window_compile_bounded: null host pointer");
  if (capacities[0] < 0 || capacities[1] < 0 || capacities[2] < 0)
    return fail(AKV_EINVAL, "akv_window_compile_bounded: negative capacity");
  Inputs in{n, birth_positions, birth_stages, transition_offsets, stage_count, transition_raw_tokens,
            transition_old_positions, transition_new_positions, visible_until, terminal_positions,
            query_start, query_end};
  // one replay: writes what fits, counts everything (a count above its
  // capacity means the arrays are incomplete)
  Sink sink = fill_sink(capacities, occurrence_raw_tokens, occurrence_positions, terminal_occurrences,
                        segment_query_starts, segment_query_ends, segment_key_offsets, segment_key_occurrences);
  sink.bounded = true;
  const int rc = run(in, sink);
  if (rc) return rc;
  counts[0] = sink.occurrences;
  counts[1] = sink.segments;
  counts[2] = sink.keys;
  counts[3] = sink.first_final;
  return AKV_OK;
}
