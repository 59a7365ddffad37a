/* llb_backend_hip.h -- the reference host's backend contract (host/llb_backend.h:1-51) on the MI355X
 * library. A C host includes this header first, then host/llb_backend.h, exactly as it includes
 * host/llb_backend_cuda.h today; the chains keep their calls unchanged:
 *
 *   llb_dptr                 u64 device address; byte offsets add to it (llb_moe_hip.h)
 *   LLB_LAUNCH(k, gx, gy, bx, &a0, &a1, ...)           -> true if queued
 *   LLB_LAUNCH_SM(k, gx, gy, bx, sm, &a0, &a1, ...)    -> true if queued, sm bytes of dynamic LDS
 *       k: a kernel looked up by name (llb_hip_module_function; the twin of cuModuleGetFunction).
 *       Each argument is the address of a host variable holding its value (a u32, a float, an
 *       llb_dptr or a by-value struct); the values are copied at the call. Launches go to the
 *       library's stream in call order, so each sees every earlier launch's writes, and they order
 *       with the llb_moe_hip_* entry points, which use the same stream.
 *   llb_alloc_zero(bytes)    -> zeroed device memory, 0 on failure
 *   llb_zero(p, bytes)       -> true if queued (stream order)
 *   llb_copy(d, s, bytes)    -> true if queued (stream order)
 *   llb_write(d, h, bytes)   -> true once host h's bytes are in d
 *   llb_read(h, p, bytes)    -> true once p's bytes are in h (after every earlier launch)
 *   llb_sync()               -> true once the queued work is done
 *   llb_dev(p)               -> the device address of a host pointer. HIP's unified addressing gives
 *       memory from hipHostMalloc (pinned, mapped: what the reference's corpus is on the CUDA side, a
 *       cuMemHostAlloc / managed allocation) the same address on the device as on the host, so this
 *       is the bit-for-bit cast the CUDA backend uses (host/llb_backend_cuda.h:221).
 *
 * The macros are C (compound-literal argument arrays, C99); the reference host is C.
 */
#ifndef LLB_BACKEND_HIP_H
#define LLB_BACKEND_HIP_H
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#include "llb_moe_hip.h"

#define LLB_LAUNCH(k, gx, gy, bx, ...) LLB_LAUNCH_SM(k, gx, gy, bx, 0, __VA_ARGS__)
#define LLB_LAUNCH_SM(k, gx, gy, bx, sm, ...)                                                        \
  ((bool)(llb_hip_launch((k), (uint32_t)(gx), (uint32_t)(gy), (uint32_t)(bx), (uint32_t)(sm),        \
                         (void*[]){__VA_ARGS__},                                                     \
                         (uint32_t)(sizeof((void*[]){__VA_ARGS__}) / sizeof(void*))) == 0))

static inline llb_dptr llb_alloc_zero(size_t bytes) { return llb_hip_alloc_zero(bytes); }
static inline bool llb_zero(llb_dptr p, size_t bytes) { return llb_hip_zero(p, bytes) == 0; }
static inline bool llb_copy(llb_dptr d, llb_dptr s, size_t bytes) { return llb_hip_copy(d, s, bytes) == 0; }
static inline bool llb_write(llb_dptr d, const void* h, size_t bytes) { return llb_hip_write(d, h, bytes) == 0; }
static inline bool llb_read(void* h, llb_dptr p, size_t bytes) { return llb_hip_read(h, p, bytes) == 0; }
static inline bool llb_sync(void) { return llb_hip_sync() == 0; }

#define llb_dev(p) ((llb_dptr)(uintptr_t)(p))
#endif
