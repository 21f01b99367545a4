// Library identity, error reporting and geometry validation.
#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace moba {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int status, const std::string& msg) {
  set_error(msg);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(MOBA_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return MOBA_OK;
}

int make_geometry(Geometry* g, int64_t batch, int64_t seq_len,
                  int64_t max_seqlen, int64_t h_q, int64_t h_kv,
                  int64_t head_dim, int64_t n_blocks, int64_t block_size,
                  int64_t slots, const int32_t* cu_seqlens) {
  if (batch <= 0 || seq_len <= 0 || h_q <= 0 || h_kv <= 0 || head_dim <= 0 ||
      block_size <= 0 || n_blocks <= 0 || slots < 0)
    return fail(MOBA_ERR_INVALID, "non-positive shape argument");
  if (h_q % h_kv != 0)
    return fail(MOBA_ERR_INVALID, "query heads " + std::to_string(h_q) +
                                      " not divisible by kv heads " +
                                      std::to_string(h_kv));
  g->rows = batch;
  g->seq_len = seq_len;
  g->packed = cu_seqlens != nullptr;
  g->rows_per_seq = g->packed ? max_seqlen : seq_len;
  if (g->packed && max_seqlen <= 0)
    return fail(MOBA_ERR_INVALID, "max_seqlen must be positive when packed");
  g->h_q = h_q;
  g->h_kv = h_kv;
  g->group = h_q / h_kv;
  g->head_dim = head_dim;
  g->n_blocks = n_blocks;
  g->block_size = block_size;
  g->slots = slots;
  if (cdiv(g->rows_per_seq, block_size) > n_blocks)
    return fail(MOBA_ERR_INVALID, "n_blocks smaller than cdiv(seq, block_size)");
  return MOBA_OK;
}

}  // namespace moba

extern "C" {

int moba_abi_version(void) { return 6; }

const char* moba_last_error(void) { return moba::g_last_error.c_str(); }

const char* moba_status_string(int status) {
  switch (status) {
    case MOBA_OK: return "ok";
    case MOBA_ERR_INVALID: return "invalid argument";
    case MOBA_ERR_UNSUPPORTED: return "unsupported configuration";
    case MOBA_ERR_LAUNCH: return "kernel launch failed";
    case MOBA_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

}  // extern "C"
