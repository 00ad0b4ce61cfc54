// Instantiations of every PoM kernel template for element type __half.
#include "agg_impl.h"
#include "scan_impl.h"
#include "gate_impl.h"
#include "heads_impl.h"
#include "features_impl.h"

namespace pom {
template hipError_t agg_fwd_t<__half>(const AggParams&, hipStream_t);
template hipError_t agg_bwd_t<__half>(const AggParams&, hipStream_t);
template hipError_t scan_fwd_t<__half>(const ScanParams&, hipStream_t);
template hipError_t scan_bwd_t<__half>(const ScanParams&, hipStream_t);
template hipError_t gate_fwd_t<__half>(const GateParams&, int, hipStream_t);
template hipError_t gate_bwd_t<__half>(const GateParams&, int, hipStream_t);
template hipError_t heads_fwd_t<__half>(const HeadsParams&, hipStream_t);
template hipError_t heads_bwd_t<__half>(const HeadsParams&, hipStream_t);
template hipError_t features_fwd_t<__half>(const FeatParams&, hipStream_t);
template hipError_t features_bwd_t<__half>(const FeatParams&, hipStream_t);
}  // namespace pom
