// static_scratch.hip - the Linear entry point that allocates nothing
// (ihip_enqueue_linear_at_static): its quantized activations live in a
// file-scope device array instead of the context's growable scratch buffer,
// for callers that cannot call hipMalloc (code under graph capture, serving
// loops, harnesses that forbid allocation). Compiled as HIP so the array is
// registered with the runtime; the kernels stay in the embedded code objects
// and take the array's device address as an argument.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "internal.h"

// the whole of the quantized activations of one call: rows * (in + in / 8)
// bytes (Q8_0 and Q8_K rows have the same size); held by every device the
// library runs on until the process ends. Host code never passes `scratch`
// itself (a host-side stand-in): only the device address that
// static_scratch_init reads for the context's device.
static __device__ __align__(256) uint8_t scratch[IHIP_STATIC_SCRATCH_BYTES];

namespace ihip {

// the one context per device whose multi-row calls may use the array: the
// first to make one, until it is destroyed. Another context's streams are not
// ordered with its stream, so its calls would race on the array unseen.
static std::mutex owners_mu;
static std::map<int, const ihip_ctx*> owners;

static bool claim(const ihip_ctx* c)
{
  std::lock_guard<std::mutex> g(owners_mu);
  auto it = owners.find(c->device);
  if (it == owners.end()) {
    owners[c->device] = c;
    return true;
  }
  return it->second == c;
}

void static_scratch_release(const ihip_ctx* c)
{
  std::lock_guard<std::mutex> g(owners_mu);
  auto it = owners.find(c->device);
  if (it != owners.end() && it->second == c) owners.erase(it);
}

int static_scratch_init(ihip_ctx* c)
{
  // with the context's device current (ihip_create): each device has its own
  // copy of the array at its own address
  // (::scratch: inside namespace ihip the bare name is the growable-scratch
  // function of the context)
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
  if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
  c->static_scratch = (uint64_t)p;
  return 0;
}

}  // namespace ihip

using namespace ihip;

extern "C" int ihip_enqueue_linear_at_static(ihip_ctx* c, uint64_t x, int64_t rows, int64_t in,
                                             int dtype, uint64_t w, int64_t out, uint64_t y,
                                             uint64_t bias, int mode)
{
  if (!c) return fail(IHIP_E_ARG, "no context");
  if (!c->static_scratch) return fail(IHIP_E_ARG, "ihip_enqueue_linear_at_static: no static scratch");
  if (!linear_ok(dtype, in) || rows < 1 || rows > 65535 || !x || !w || !y)
    return fail(IHIP_E_ARG, "ihip_enqueue_linear_at_static: " + std::to_string(rows) + " rows of " +
                                std::to_string(in) + " dtype " + std::to_string(dtype));
  LinearCall k;
  k.x = x; k.rows = rows; k.in = in; k.dtype = dtype; k.w = w; k.out = out; k.y = y;
  k.bias = bias; k.mode = mode; k.no_alloc = true;
  const int kind = q8_kind(dtype);
  // one row quantizes its groups in the GEMV's registers; several rows are
  // quantized once into the array, as the context's scratch would hold them
  if ((mode & 1) == IHIP_MODE_Q8 && !(mode & IHIP_MODE_XQ) && kind >= 0 && rows > 1) {
    if ((uint64_t)rows * q8_row_bytes(in) > IHIP_STATIC_SCRATCH_BYTES)
      return fail(IHIP_E_NOMEM, "ihip_enqueue_linear_at_static: " + std::to_string(rows) +
                                    " rows of " + std::to_string(in) + " need more than the " +
                                    std::to_string(IHIP_STATIC_SCRATCH_BYTES) +
                                    " bytes of static scratch");
    if (!claim(c))
      return fail(IHIP_E_ARG, "ihip_enqueue_linear_at_static: the static scratch of device " +
                                  std::to_string(c->device) +
                                  " belongs to another context (calls of two contexts would race)");
    int rc = enqueue_quantize(c, x, rows, in, kind, c->static_scratch);
    if (rc) return rc;
    k.xq = c->static_scratch;
  }
  return enqueue_linear(c, k);
}
