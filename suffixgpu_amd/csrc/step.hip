// Fused decode step (suffix_gpu/proposer.py:186-327): the local kernel on
// the caller's stream, the global kernel on the side stream; rows meet in
// the workspace and the later of the two writes the row's draft.

#include "launch.h"
#include "step_ws.h"

using namespace sfx;

extern "C" size_t sfx_step_workspace_size(const sfx_params* p,
                                          int64_t batch) {
  if (!p || batch < 0) return 0;
  return step_ws_layout(*p, batch, nullptr, nullptr);
}

extern "C" int sfx_propose_step(const sfx_params* p, const sfx_index* ix,
                                const sfx_batch* bt, int32_t* draft,
                                int32_t* num_valid, int32_t* new_counts,
                                void* workspace, size_t workspace_bytes,
                                hipStream_t stream, hipStream_t side_stream) {
  if (!p || !bt || !draft || !num_valid) return SFX_EINVAL;
  int rc = check_local(*p, *bt);
  if (rc) return rc;
  if (bt->sampled && bt->limit < 0) return SFX_EINVAL;
  const bool global_on = ix != nullptr;
  if (global_on) {
    rc = check_global(*p, *ix);
    if (rc) return rc;
  }
  StepWs ws = {};
  if (global_on) {
    const size_t need = step_ws_layout(*p, bt->batch, nullptr, nullptr);
    if (!workspace || workspace_bytes < need) return SFX_EINVAL;
    step_ws_layout(*p, bt->batch, workspace, &ws);
  }
  // The global kernel reads each row's tail through the step's sampled ids
  // (pick.h updated_token), so it does not wait for the local kernel's
  // scatter; the two only meet in the workspace.
  rc = local_step(*p, *bt, global_on, draft, num_valid, new_counts, ws,
                  stream);
  if (rc) return rc;
  if (global_on) {
    rc = global_step(*p, *ix, *bt, draft, num_valid, ws,
                     side_stream ? side_stream : stream);
    if (rc) return rc;
  }
  return 0;
}
