// drv_kernels.hip -- a code object for the standalone C host (moe_layer_drv.c), launched by name through
// LLB_LAUNCH (include/llb_backend_hip.h): it stages the token rows the generator wrote into the
// buffers the layer reads, the role the reference host's own kernels play before llb_moe_run.
#include <hip/hip_runtime.h>
#include <stdint.h>

struct DrvSpan {  // a by-value argument, as the reference passes Q8Cat
  const float* src;
  float* dst;
  uint32_t n;
  uint32_t pad;
};

// grid (ceil(max n / 256), 2): y = 0 copies span a, y = 1 span b, each element times scale
extern "C" __global__ void __launch_bounds__(256) llb_drv_stage(DrvSpan a, DrvSpan b, float scale) {
  const DrvSpan s = blockIdx.y ? b : a;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < s.n) s.dst[i] = s.src[i] * scale;
}
