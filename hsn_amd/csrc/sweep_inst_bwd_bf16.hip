// The kernels of the backward sweep, bf16 storage and int32 slots, instantiated in a
// translation unit of their own so the sweeps' kernels compile in parallel.
#define HSN_SWEEP_INSTANTIATE
#include "sweep.cuh"

namespace hsn {
template hipError_t launch_bwd<bf16_t, Packed32, true>(const BwdArgs&, int, size_t, hipStream_t);
}  // namespace hsn
