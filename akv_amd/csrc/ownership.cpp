// Host ownership planner of a request's prefill forwards: which occurrence
// versions need a KV page, which of them an existing owner row already holds,
// the copies that fill the rest, and after binding the forward's slots, the
// successor ownership state and the private pages to retire.
//
// Same decisions and error messages as plan_occurrence_materialization and
// OccurrenceState.advance
// (akv/system/sglang/srt/context_system/occurrence.py:341-466, 632-755),
// as linear passes over plain arrays behind the C ABI.  Everything here is
// index bookkeeping on owner *rows*; slot values stay on the device and are
// resolved by one batched gather launch (akv_gather_slots).
//
// Owner rows of the plan address canonical[0:n] ++ terminal[0:n] of the raw
// tokens (row r = canonical version of raw r, row n + r = terminal version).
// Rows of the advance address the request's slot sequence
// old[0:R] ++ query[0:q] ++ extra[0:A].
#include <algorithm>
#include <cstdint>
#include <string>
#include <vector>

#include "abi_common.h"

namespace {

constexpr uint8_t kRead = 1, kNeed = 2, kPublish = 4;

bool any_null(std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (!p) return true;
  return false;
}

}  // namespace

extern "C" int akv_plan_ownership(int64_t n, int64_t query_start, int64_t query_end, int64_t exact_prefix_len,
                                  int64_t occurrence_count, const int32_t* occurrence_raw_tokens,
                                  const int32_t* occurrence_positions, const int32_t* terminal_occurrences,
                                  int64_t key_count, const int32_t* key_occurrences,
                                  const int32_t* canonical_positions, const uint8_t* canonical_present,
                                  const uint8_t* canonical_owned, const uint8_t* terminal_present,
                                  const uint8_t* terminal_keep, int64_t* source_rows, int64_t* allocated,
                                  int64_t* copy_source_rows, int32_t* copy_position_pairs,
                                  int64_t* selected_terminal, uint8_t* read_cached, uint8_t* repositioned_cached,
                                  int64_t* allocated_count) {
  using namespace akv;
  if (!(0 <= exact_prefix_len && exact_prefix_len <= query_start && query_start < query_end && query_end <= n))
    return fail(AKV_EINVAL, "Invalid occurrence ownership/query boundaries");
  if (occurrence_count < n || key_count < 0)
    return fail(AKV_EINVAL, "akv_plan_ownership: the window does not cover the raw prompt");
  if (any_null({occurrence_raw_tokens, occurrence_positions, terminal_occurrences, terminal_keep, source_rows,
                allocated, copy_source_rows, copy_position_pairs, selected_terminal, read_cached,
                repositioned_cached, allocated_count}) ||
      (key_count && !key_occurrences) ||
      (query_start && any_null({canonical_positions, canonical_present, canonical_owned, terminal_present})))
    return fail(AKV_EINVAL, "akv_plan_ownership: null host pointer");

  // per raw token: canonical presence / ownership / position, terminal owner
  std::vector<uint8_t> have(n, 0), mine(n, 0), tlive(n, 0);
  std::vector<int32_t> cpos(n), tpos(n);
  for (int64_t t = 0; t < n; ++t) {
    const int32_t term = terminal_occurrences[t];
    if (term < 0 || term >= occurrence_count || occurrence_raw_tokens[term] != t)
      return fail(AKV_EINVAL, "akv_plan_ownership: terminal occurrence of raw token %lld is invalid",
                  static_cast<long long>(t));
    if (occurrence_raw_tokens[t] != t)
      return fail(AKV_EINVAL, "akv_plan_ownership: occurrences [0, n) must be the birth versions");
    tpos[t] = occurrence_positions[term];
    cpos[t] = occurrence_positions[t];
  }
  for (int64_t t = 0; t < query_start; ++t) {
    have[t] = canonical_present[t] != 0;
    mine[t] = canonical_owned[t] != 0;
    tlive[t] = terminal_present[t] != 0;
    cpos[t] = canonical_positions[t];
  }
  for (int64_t t = query_start; t < query_end; ++t) have[t] = mine[t] = 1;

  std::vector<uint8_t> flag(occurrence_count, 0);
  for (int64_t k = 0; k < key_count; ++k) {
    const int32_t o = key_occurrences[k];
    if (o < 0 || o >= occurrence_count) return fail(AKV_EINVAL, "akv_plan_ownership: segment key out of range");
    flag[o] |= kRead | kNeed;
  }
  for (int64_t t = query_start; t < query_end; ++t) flag[t] |= kNeed;
  for (int64_t t = 0; t < query_end; ++t) {
    selected_terminal[t] = -1;
    if (terminal_keep[t]) {
      const int32_t o = terminal_occurrences[t];
      flag[o] |= kNeed | kPublish;
      selected_terminal[t] = o;
    }
  }
  std::fill(read_cached, read_cached + n, 0);
  std::fill(repositioned_cached, repositioned_cached + n, 0);

  int64_t a = 0;
  std::vector<int32_t> lost;
  for (int64_t o = 0; o < occurrence_count; ++o) {
    source_rows[o] = -1;
    const uint8_t f = flag[o];
    if (!(f & kNeed)) continue;
    const int32_t r = occurrence_raw_tokens[o];
    const int32_t p = occurrence_positions[o];
    if (r < 0 || r >= n) return fail(AKV_EINVAL, "akv_plan_ownership: occurrence raw token out of range");
    if ((f & kRead) && r < query_start) {
      read_cached[r] = 1;
      if (p != cpos[r]) repositioned_cached[r] = 1;
    }
    const bool at_terminal = tlive[r] && tpos[r] == p;
    const bool at_canonical = have[r] && cpos[r] == p;
    // a borrowed page past the exact prefix never becomes the published
    // owner of this version, even at the same position
    const bool must_own = (f & kPublish) && r >= exact_prefix_len && !mine[r] && !at_terminal;
    if (at_terminal) {
      source_rows[o] = n + r;
    } else if (at_canonical && !must_own) {
      source_rows[o] = r;
    } else {
      allocated[a] = o;
      if (have[r]) {  // the canonical owner is preferred as the copy source
        copy_source_rows[a] = r;
        copy_position_pairs[2 * a] = cpos[r];
      } else if (tlive[r]) {
        copy_source_rows[a] = n + r;
        copy_position_pairs[2 * a] = tpos[r];
      } else {
        lost.push_back(r);
        copy_source_rows[a] = -1;
        copy_position_pairs[2 * a] = 0;
      }
      copy_position_pairs[2 * a + 1] = p;
      ++a;
    }
  }
  if (!lost.empty()) {
    std::sort(lost.begin(), lost.end());
    lost.erase(std::unique(lost.begin(), lost.end()), lost.end());
    std::string list = "[";
    for (size_t i = 0; i < lost.size(); ++i) list += (i ? ", " : "") + std::to_string(lost[i]);
    list += "]";
    return fail(AKV_EINVAL, "Occurrence recovery required for raw tokens %s", list.c_str());
  }
  *allocated_count = a;
  return AKV_OK;
}

extern "C" int akv_advance_ownership(
    int64_t n, int64_t start, int64_t end, int64_t old_count, int64_t query_count, int64_t extra_count,
    const uint8_t* owned, const int64_t* canonical_rows, const int64_t* terminal_rows,
    const int32_t* canonical_positions, int32_t track_swa, const uint8_t* swa_resident, int64_t occurrence_count,
    const int32_t* occurrence_positions, const int32_t* terminal_occurrences, const int64_t* source_rows,
    const int64_t* allocated, const int64_t* copy_source_rows, const int64_t* selected_terminal,
    const int32_t* visible_until, int64_t* occurrence_rows, int64_t* copy_source_index,
    int64_t* copy_destination_index, int64_t* successor_rows, int64_t* retired_rows, int64_t* unused_swa_rows,
    uint8_t* next_owned, int64_t* next_canonical, int64_t* next_terminal, int32_t* next_positions,
    uint8_t* next_swa, uint8_t* retired_swa, int64_t* counts) {
  using namespace akv;
  if (!(0 <= start && start < end && end <= n) || old_count < 0 || extra_count < 0 || occurrence_count < n)
    return fail(AKV_EINVAL, "akv_advance_ownership: invalid window bounds");
  if (query_count != end - start) return fail(AKV_EINVAL, "Context admission does not cover the selected window");
  if (any_null({occurrence_positions, terminal_occurrences, source_rows, selected_terminal, visible_until,
                occurrence_rows, successor_rows, retired_rows, next_owned, next_canonical, next_terminal,
                next_positions, counts}) ||
      (old_count && !owned) || (start && any_null({canonical_rows, terminal_rows, canonical_positions})) ||
      (extra_count && any_null({allocated, copy_source_rows, copy_source_index, copy_destination_index})) ||
      (track_swa && (any_null({next_swa, retired_swa, unused_swa_rows}) || (old_count && !swa_resident))))
    return fail(AKV_EINVAL, "akv_advance_ownership: null host pointer");
  const int64_t total = old_count + query_count + extra_count;
  // owner row of canonical[i] (i < n) or terminal[i - n]
  auto by_row = [&](int64_t i) -> int64_t {
    if (i < n) {
      if (i < start) return canonical_rows[i];
      if (i < end) return old_count + (i - start);
      return -1;
    }
    const int64_t t = i - n;
    return t < start ? terminal_rows[t] : -1;
  };
  for (int64_t t = 0; t < start; ++t)
    if (canonical_rows[t] < -1 || canonical_rows[t] >= old_count || terminal_rows[t] < -1 ||
        terminal_rows[t] >= old_count)
      return fail(AKV_EINVAL, "akv_advance_ownership: state rows out of range");
  for (int64_t t = 0; t < end; ++t)
    if (terminal_occurrences[t] < 0 || terminal_occurrences[t] >= occurrence_count)
      return fail(AKV_EINVAL, "akv_advance_ownership: terminal occurrence out of range");

  std::vector<int64_t> occ(occurrence_count);
  for (int64_t o = 0; o < occurrence_count; ++o) {
    const int64_t s = source_rows[o];
    if (s < -1 || s >= 2 * n) return fail(AKV_EINVAL, "akv_advance_ownership: plan source row out of range");
    occ[o] = -1;
    if (s >= 0) {
      occ[o] = by_row(s);
      if (occ[o] < 0) return fail(AKV_EINVAL, "Context ownership plan references a missing source");
    }
  }
  for (int64_t j = 0; j < extra_count; ++j) {
    if (allocated[j] < 0 || allocated[j] >= occurrence_count)
      return fail(AKV_EINVAL, "akv_advance_ownership: allocated occurrence out of range");
    occ[allocated[j]] = old_count + query_count + j;
  }
  for (int64_t j = 0; j < extra_count; ++j) {
    const int64_t s = copy_source_rows[j];
    const int64_t from = (s >= 0 && s < 2 * n) ? by_row(s) : -1;
    if (from < 0) return fail(AKV_EINVAL, "Context copy references a missing canonical source");
    copy_source_index[j] = from;
    copy_destination_index[j] = occ[allocated[j]];
  }

  std::vector<uint8_t> swa;
  int64_t unused = 0;
  if (track_swa) {
    swa.assign(total, 1);
    std::copy(swa_resident, swa_resident + old_count, swa.begin());
    // sources are canonical / terminal rows, never this forward's fresh rows
    for (int64_t j = 0; j < extra_count; ++j) swa[copy_destination_index[j]] = swa[copy_source_index[j]];
    for (int64_t j = 0; j < extra_count; ++j)
      if (!swa[copy_destination_index[j]]) unused_swa_rows[unused++] = copy_destination_index[j];
  }

  std::vector<uint8_t> live(total, 0);
  for (int64_t t = 0; t < end; ++t) {
    const int64_t chosen = selected_terminal[t];
    if (chosen < -1 || chosen >= occurrence_count)
      return fail(AKV_EINVAL, "akv_advance_ownership: selected terminal occurrence out of range");
    const int64_t term = chosen >= 0 ? occ[chosen] : -1;
    const int32_t pos = t < start ? canonical_positions[t] : occurrence_positions[t];
    int64_t canon = by_row(t);
    // a same-position terminal copy is bit-identical: later reads use it
    if (term >= 0 && pos == occurrence_positions[terminal_occurrences[t]]) canon = term;
    // only a source some later query of the prompt reads stays canonical
    if (end == n || visible_until[t] <= end) canon = -1;
    next_terminal[t] = term;
    next_canonical[t] = canon;
    next_positions[t] = pos;
    if (term >= 0) live[term] = 1;
    if (canon >= 0) live[canon] = 1;
  }
  std::vector<int64_t> remap(total, -1);
  int64_t kept = 0, retired = 0;
  for (int64_t i = 0; i < total; ++i) {
    const bool mine = i < old_count ? owned[i] != 0 : true;
    if (live[i]) {
      remap[i] = kept;
      successor_rows[kept] = i;
      next_owned[kept] = mine;
      if (track_swa) next_swa[kept] = swa[i];
      ++kept;
    } else if (mine) {
      retired_rows[retired] = i;
      if (track_swa) retired_swa[retired] = swa[i];
      ++retired;
    }
  }
  for (int64_t t = 0; t < end; ++t) {
    if (next_canonical[t] >= 0) next_canonical[t] = remap[next_canonical[t]];
    if (next_terminal[t] >= 0) next_terminal[t] = remap[next_terminal[t]];
  }
  for (int64_t o = 0; o < occurrence_count; ++o) occurrence_rows[o] = occ[o] < 0 ? 0 : occ[o];
  counts[0] = kept;
  counts[1] = retired;
  counts[2] = unused;
  return AKV_OK;
}
