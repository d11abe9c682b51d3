// Kernel timing hook (msa_profile_begin / msa_profile_end in include/msa_mi355x.h).
//
// While armed, the attention entry points bracket each kernel launch with a pair of
// HIP events recorded on the launch stream; msa_profile_end waits for them and sums
// the durations per kernel kind. Disarmed, a launch site costs one relaxed atomic load.
#pragma once
#include <hip/hip_runtime.h>

namespace msa {

// Kernel kinds, in the order msa_profile_end reports them.
enum ProfKind {
  kProfFwdPlan = 0,        // kv_chunk_bounds + kv_item_scan of the forward
  kProfFwdPartial,         // attn_fwd_partial_kernel
  kProfFwdCombine,         // attn_fwd_combine
  kProfBwdPlan,            // kv_chunk_bounds + kv_item_scan of the backward (both plans)
  kProfBwdCenter,          // kv_bwd_center
  kProfBwdStats,           // kv_bwd_stats_kernel
  kProfBwdStatsCombine,    // kv_bwd_stats_combine
  kProfBwdMain,            // kv_bwd_main_kernel
  kProfBwdAccumulate,      // kv_bwd_accumulate
  kProfBwdDqCombine,       // kv_bwd_dq_combine
  kProfKinds
};

bool prof_armed();
int prof_open(int kind, hipStream_t st);  // records a start event; -1 when not recording
void prof_close(int pair, hipStream_t st);  // records the matching stop event

// Brackets the launches issued during its lifetime.
class ProfScope {
 public:
  ProfScope(int kind, hipStream_t st) : st_(st), pair_(prof_armed() ? prof_open(kind, st) : -1) {}
  ~ProfScope() {
    if (pair_ >= 0) prof_close(pair_, st_);
  }
  ProfScope(const ProfScope&) = delete;
  ProfScope& operator=(const ProfScope&) = delete;

 private:
  hipStream_t st_;
  int pair_;
};

}  // namespace msa
