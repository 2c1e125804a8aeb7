// placeholder, replaced by the chunked prefill
#include "gdn_common.h"
#include "gdn_host.h"
using namespace gdn;
extern "C" int64_t gdn_prefill_workspace_size(int, int64_t, int, int, int, int) { return 0; }
extern "C" int gdn_prefill_chunked(const void*, const void*, const void*, const void*, const void*, int,
                                   const float*, const float*, int, const float*, float*, void*, int,
                                   const int32_t*, int, int64_t, int, int, int, int, void*, int64_t, void*) {
    return fail(GDN_EUNSUPPORTED, "gdn_prefill_chunked: not built yet");
}
