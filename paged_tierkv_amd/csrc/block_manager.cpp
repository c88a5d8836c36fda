// Host-side BlockManager and the library's error plumbing (C ABI).
//
// Same allocation order, states and error messages as the reference's
// pybind11 BlockManager (csrc/block_manager.cpp:22-124):
//   * the free list is a stack filled total-1 .. 0, so allocation hands out
//     0, 1, 2, ... on a fresh manager and reuses freed ids LIFO;
//   * a new block is HOT with logical id = the sequence's current length;
//   * free_sequence returns the ids in logical order, no-op when unknown;
//   * update_block_state rejects an unknown sequence, a logical id out of
//     range and a state outside {0, 1, 2}.
// Sequences live in a hash map of dense vectors; the physical ids and the
// states are kept in two parallel arrays so the getters are plain copies.

#include <cstdint>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tierkv_hip.h"

namespace tierkv {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

}  // namespace tierkv

struct tierkv_block_manager {
  struct Seq {
    std::vector<int32_t> physical;
    std::vector<int32_t> states;
  };
  int32_t total_blocks = 0;
  std::vector<int32_t> free_list;
  std::unordered_map<int32_t, Seq> seqs;
};

using tierkv::set_error;
using tierkv::clear_error;

static int32_t state_error(const char* msg) {
  set_error(msg);
  return TIERKV_ERR_STATE;
}

extern "C" const char* tierkv_last_error(void) { return tierkv::g_last_error.c_str(); }

extern "C" int32_t tierkv_abi_version(void) { return 1; }

extern "C" int32_t tierkv_bm_create(int32_t total_blocks, tierkv_block_manager** out) {
  clear_error();
  if (!out) {
    set_error("null output pointer");
    return TIERKV_ERR_INVALID;
  }
  *out = nullptr;
  if (total_blocks <= 0) return state_error("total_blocks must be positive");
  tierkv_block_manager* bm = new (std::nothrow) tierkv_block_manager();
  if (!bm) return state_error("out of host memory");
  bm->total_blocks = total_blocks;
  bm->free_list.reserve(static_cast<size_t>(total_blocks));
  for (int32_t i = total_blocks - 1; i >= 0; --i) bm->free_list.push_back(i);
  *out = bm;
  return TIERKV_OK;
}

extern "C" void tierkv_bm_destroy(tierkv_block_manager* bm) { delete bm; }

extern "C" int32_t tierkv_bm_allocate_block(tierkv_block_manager* bm, int32_t seq_id, int32_t* physical_idx) {
  clear_error();
  if (!bm || !physical_idx) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  if (bm->free_list.empty()) return state_error("No free physical blocks available.");
  const int32_t phys = bm->free_list.back();
  bm->free_list.pop_back();
  auto& s = bm->seqs[seq_id];
  s.physical.push_back(phys);
  s.states.push_back(0);
  *physical_idx = phys;
  return TIERKV_OK;
}

extern "C" int32_t tierkv_bm_free_sequence(tierkv_block_manager* bm, int32_t seq_id) {
  clear_error();
  if (!bm) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  auto it = bm->seqs.find(seq_id);
  if (it == bm->seqs.end()) return TIERKV_OK;
  for (int32_t phys : it->second.physical) bm->free_list.push_back(phys);
  bm->seqs.erase(it);
  return TIERKV_OK;
}

extern "C" int32_t tierkv_bm_update_block_state(tierkv_block_manager* bm, int32_t seq_id, int32_t logical_id,
                                                int32_t state) {
  clear_error();
  if (!bm) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  auto it = bm->seqs.find(seq_id);
  if (it == bm->seqs.end()) return state_error("Sequence not found for state update.");
  auto& s = it->second;
  if (logical_id < 0 || logical_id >= static_cast<int32_t>(s.states.size()))
    return state_error("Logical block ID out of range.");
  if (state < 0 || state > 2) return state_error("Invalid BlockState value.");
  s.states[static_cast<size_t>(logical_id)] = state;
  return TIERKV_OK;
}

extern "C" int32_t tierkv_bm_set_block_states(tierkv_block_manager* bm, int32_t seq_id, const int32_t* states,
                                              int32_t n) {
  clear_error();
  if (!bm || (n > 0 && !states)) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  auto it = bm->seqs.find(seq_id);
  if (it == bm->seqs.end()) return state_error("Sequence not found for state update.");
  auto& s = it->second;
  if (n < 0 || n > static_cast<int32_t>(s.states.size())) return state_error("Logical block ID out of range.");
  for (int32_t i = 0; i < n; ++i)
    if (states[i] < 0 || states[i] > 2) return state_error("Invalid BlockState value.");
  std::memcpy(s.states.data(), states, sizeof(int32_t) * static_cast<size_t>(n));
  return TIERKV_OK;
}

extern "C" int32_t tierkv_bm_num_blocks(const tierkv_block_manager* bm, int32_t seq_id, int32_t* n) {
  clear_error();
  if (!bm || !n) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  auto it = bm->seqs.find(seq_id);
  *n = (it == bm->seqs.end()) ? 0 : static_cast<int32_t>(it->second.physical.size());
  return TIERKV_OK;
}

static int32_t copy_out(const std::vector<int32_t>* src, int32_t* out, int32_t capacity, int32_t* n) {
  const int32_t count = src ? static_cast<int32_t>(src->size()) : 0;
  if (n) *n = count;
  if (count > 0 && out && capacity > 0) {
    const int32_t m = count < capacity ? count : capacity;
    std::memcpy(out, src->data(), sizeof(int32_t) * static_cast<size_t>(m));
  }
  return TIERKV_OK;
}

extern "C" int32_t tierkv_bm_get_physical_indices(const tierkv_block_manager* bm, int32_t seq_id, int32_t* out,
                                                  int32_t capacity, int32_t* n) {
  clear_error();
  if (!bm) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  auto it = bm->seqs.find(seq_id);
  return copy_out(it == bm->seqs.end() ? nullptr : &it->second.physical, out, capacity, n);
}

extern "C" int32_t tierkv_bm_get_states(const tierkv_block_manager* bm, int32_t seq_id, int32_t* out,
                                        int32_t capacity, int32_t* n) {
  clear_error();
  if (!bm) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  auto it = bm->seqs.find(seq_id);
  return copy_out(it == bm->seqs.end() ? nullptr : &it->second.states, out, capacity, n);
}

extern "C" int32_t tierkv_bm_num_free(const tierkv_block_manager* bm, int32_t* n) {
  clear_error();
  if (!bm || !n) {
    set_error("null pointer");
    return TIERKV_ERR_INVALID;
  }
  *n = static_cast<int32_t>(bm->free_list.size());
  return TIERKV_OK;
}
