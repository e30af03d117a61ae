// ABI plumbing shared by all entry points: version, status strings, layout validation.
#include "common.h"

namespace oscar {

int make_layout(const oscar_layout* in, Layout* out) {
  if (!in || !out) return OSCAR_E_NULL;
  if (in->head_dim != kHeadDim) return OSCAR_E_UNSUPPORTED;
  const int h = in->kv_heads, bp = in->physical_block_tokens, bk = in->kernel_block_tokens;
  if (h <= 0 || bp <= 0 || bk < 32 || (bk & (bk - 1)) || bp % bk) return OSCAR_E_LAYOUT;
  const int vector = in->head_dim / 4 + 4;
  const int slot = ((2 * vector + 31) / 32) * 32;
  if (in->vector_bytes != vector || in->slot_bytes != slot) return OSCAR_E_LAYOUT;
  if (in->sink_tokens < 0 || in->recent_tokens < 0 || in->ring_tokens <= 0) return OSCAR_E_LAYOUT;
  const int64_t page = static_cast<int64_t>(bp) * h * in->head_dim * 2;
  if (in->stripe_page_bytes != page) return OSCAR_E_LAYOUT;
  if (static_cast<int64_t>(bp) * h * slot > page) return OSCAR_E_LAYOUT;
  const int64_t window = static_cast<int64_t>(in->sink_tokens + in->ring_tokens) * 2 * h *
                         in->head_dim * 2;
  if (window > page) return OSCAR_E_LAYOUT;
  out->page_bytes = page;
  out->head_dim = in->head_dim;
  out->kv_heads = h;
  out->bp = bp;
  out->bk = bk;
  int shift = 0;
  while ((1 << shift) < bk) ++shift;
  out->bk_shift = shift;
  out->bpp = bp / bk;
  out->slot_bytes = slot;
  out->vector_bytes = vector;
  out->sink = in->sink_tokens;
  out->recent = in->recent_tokens;
  out->ring = in->ring_tokens;
  out->bpp_div = make_fastdiv(static_cast<uint32_t>(out->bpp));
  out->ring_div = make_fastdiv(static_cast<uint32_t>(out->ring));
  out->bp_div = make_fastdiv(static_cast<uint32_t>(bp));
  return OSCAR_OK;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace oscar

extern "C" int oscar_abi_version(void) { return OSCAR_ABI_VERSION; }

extern "C" const char* oscar_status_string(int status) {
  switch (status) {
    case OSCAR_OK: return "ok";
    case OSCAR_E_NULL: return "a required pointer is NULL";
    case OSCAR_E_SHAPE: return "inconsistent or unsupported sizes/strides";
    case OSCAR_E_LAYOUT: return "invalid cache layout";
    case OSCAR_E_ALIGN: return "pointer or stride alignment not supported";
    case OSCAR_E_UNSUPPORTED: return "request outside this build's coverage";
    case OSCAR_E_SCRATCH:
      return "request exceeds the fixed scratch array of an allocation-free entry point";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
