// Library-wide C-ABI entries: error text and version.
#include <string>

#include "si_status.h"

namespace si {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

}  // namespace si

extern "C" const char* si_last_error(void) { return si::g_last_error.c_str(); }

// Bumped whenever an entry point's signature or semantics change.
extern "C" int si_abi_version(void) { return 8; }

// The fused indexer keeps every selection buffer in LDS, so the top-k entry
// needs no device workspace at any size.  Kept so callers that size a
// workspace (the chunk_s x chunk_t score tile of the reference driver) can ask.
extern "C" size_t si_indexer_topk_workspace_bytes(int64_t B, int64_t S, int64_t T, int64_t H, int64_t D,
                                                   int64_t top_k) {
  (void)B; (void)S; (void)T; (void)H; (void)D; (void)top_k;
  return 0;
}
