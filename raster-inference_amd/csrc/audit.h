// Challenger-side comparison of checkpoint trace artifacts: parsing a
// claimed trace (shared/api/audit.rs:34-82 ClaimedTrace), locating the first
// divergence from a replay (runtime/roles/challenger.rs:136-183) and mapping
// it to the raster detour spec (challenger.rs:185-210). Host code only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace det_audit {

// A claimed trace that is not a JSON array of single-key
// {checkpoint_id: "commitment"} objects.
struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// One committed checkpoint with its 1-based occurrence among the entries of
// the same checkpoint id (ClaimedTraceEntry, audit.rs:16-24).
struct Entry {
  uint64_t entry_index;
  std::string checkpoint_id;
  uint64_t occurrence;
  std::string commitment;
};

// ClaimedTrace::from_json_bytes: any JSON text (RFC 8259, arrays and
// objects nested less than 128 deep, UTF-8 strings) whose value is such an
// array. Throws Error.
std::vector<Entry> parse_trace(const char* bytes, size_t n);

// ClaimedTrace::from_value of a collector's committed (checkpoint_id,
// commitment) pairs in commit order.
std::vector<Entry> entries_of(const std::vector<std::pair<std::string, std::string>>& committed);

// A JSON string literal as serde_json writes it: quote, backslash and
// control characters escaped, every other byte copied.
std::string json_quote(const std::string& v);

// CheckpointDivergence (audit.rs:85-110); a has_* flag false is None.
struct Divergence {
  uint64_t entry_index = 0;
  std::string checkpoint_id;
  uint64_t occurrence = 0;
  bool has_claimed_checkpoint_id = false;
  std::string claimed_checkpoint_id;
  bool has_claimed_commitment = false;
  std::string claimed_commitment;
  bool has_replayed_commitment = false;
  std::string replayed_commitment;
};

// locate_first_divergence: false when both sequences agree entirely.
bool first_divergence(const std::vector<Entry>& claimed, const std::vector<Entry>& replayed, Divergence* out);

// detour_spec_for: the --raster-at spec of the divergent routine occurrence
// ("id" for occurrence 1, else "id:occurrence"), or "" for a structural
// divergence or a routine without a raster detour.
std::string detour_spec(const Divergence& d);

// The audit outcome as compact JSON: {"diverged":false} or
// {"diverged":true,"divergence":{...},"detour":"spec"|null}, the divergence
// object with the fields of CheckpointDivergence in declaration order and
// the None ones left out (its serde form).
std::string outcome_json(const std::vector<Entry>& claimed, const std::vector<Entry>& replayed, bool* diverged);

}  // namespace det_audit
