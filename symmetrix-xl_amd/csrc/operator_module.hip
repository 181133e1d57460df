// One M0 or R0 operator module (a gfx950 code object, hipcc --genco): the
// identity symbols and kernels the reference's OperatorModule::load reads
// (jit_operator_module.cpp:236-373), over the kernels of operator_module.hpp.
//
// Configured by macros (the Makefile's -D flags for the compiled shapes, or
// the wrapper that symmetrix/operator_modules.py renders for a contract):
//   SMX_OPMOD_KIND        1 (M0) or 2 (R0)
//   SMX_OPMOD_CHANNELS    C
//   SMX_OPMOD_LMAX        edge l_max (input harmonics (l_max+1)^2)
//   SMX_OPMOD_TABLE       M0: the monomial table type (NOUT, NT, offset[], terms[])
//   SMX_OPMOD_CORRELATION M0: the product-basis correlation order
//   SMX_OPMOD_ARTIFACT, SMX_OPMOD_STRUCTURE, SMX_OPMOD_TARGET  identity strings
#include <hip/hip_runtime.h>

#include "operator_module.hpp"
#include "product_tables.hpp"

#ifndef SMX_OPMOD_KIND
#error "SMX_OPMOD_KIND is not defined"
#endif
#ifndef SMX_OPMOD_TARGET
#define SMX_OPMOD_TARGET "gfx950"
#endif

namespace {
constexpr int kChannels = SMX_OPMOD_CHANNELS;
constexpr int kHarmonics = (SMX_OPMOD_LMAX + 1) * (SMX_OPMOD_LMAX + 1);
#if SMX_OPMOD_KIND == 1
using Table = SMX_OPMOD_TABLE;
static_assert(Table::available, "no monomial table for this module");
constexpr unsigned kCapabilities = SYMMETRIX_JIT_OPERATOR_M0_FORWARD_V1 | SYMMETRIX_JIT_OPERATOR_M0_REVERSE_V1 |
                                   SYMMETRIX_JIT_OPERATOR_M0_ALIAS_SAFE_V1 |
                                   SYMMETRIX_JIT_OPERATOR_M0_SCALE_ADJOINT_V1 |
                                   SYMMETRIX_JIT_OPERATOR_M0_RESPONSE_REVERSE_V1;
constexpr int kInputs = kHarmonics, kOutputs = Table::NOUT, kCorrelation = SMX_OPMOD_CORRELATION,
              kTerms = Table::NT;
#else
constexpr unsigned kCapabilities =
    SYMMETRIX_JIT_OPERATOR_R0_DENSITY_PREPARE_V1 | SYMMETRIX_JIT_OPERATOR_R0_FORWARD_V1 |
    SYMMETRIX_JIT_OPERATOR_R0_REVERSE_PREPARE_V1 | SYMMETRIX_JIT_OPERATOR_R0_COORDINATE_REVERSE_V1 |
    SYMMETRIX_JIT_OPERATOR_R0_COMPACT_GEOMETRY_V1 | SYMMETRIX_JIT_OPERATOR_R0_PRECOMPUTED_SCALE_V1 |
    SYMMETRIX_JIT_OPERATOR_R0_RECEIVER_BATCH_V1;
// the scalar-source R0 contract: one identity coupling term per harmonic
constexpr int kInputs = kHarmonics, kOutputs = kHarmonics, kCorrelation = 1, kTerms = kHarmonics;
#endif
}  // namespace

extern "C" {
__device__ __constant__ unsigned int symmetrix_operator_abi_version_v1 = SYMMETRIX_JIT_OPERATOR_ABI_VERSION_V1;
__device__ __constant__ unsigned int symmetrix_operator_kind_v1 = SMX_OPMOD_KIND;
__device__ __constant__ unsigned int symmetrix_operator_scalar_kind_v1 = SYMMETRIX_JIT_OPERATOR_SCALAR_FLOAT32_V1;
__device__ __constant__ unsigned int symmetrix_operator_scalar_size_v1 = sizeof(float);
__device__ __constant__ unsigned int symmetrix_operator_capabilities_v1 = kCapabilities;
__device__ __constant__ int symmetrix_operator_input_components_v1 = kInputs;
__device__ __constant__ int symmetrix_operator_output_components_v1 = kOutputs;
__device__ __constant__ int symmetrix_operator_correlation_v1 = kCorrelation;
__device__ __constant__ int symmetrix_operator_term_count_v1 = kTerms;
__device__ __constant__ int symmetrix_operator_threads_v1 = smx::opmod::kThreads;
__device__ __constant__ char symmetrix_operator_artifact_id_v1[] = SMX_OPMOD_ARTIFACT;
__device__ __constant__ char symmetrix_operator_structure_fingerprint_v1[] = SMX_OPMOD_STRUCTURE;
__device__ __constant__ char symmetrix_operator_target_v1[] = SMX_OPMOD_TARGET;

#if SMX_OPMOD_KIND == 1
__global__ __launch_bounds__(smx::opmod::kThreads) void symmetrix_m0_forward_v1(SymmetrixJitM0ArgsV1 args) {
    smx::opmod::m0_forward<kChannels, kInputs, Table>(args);
}
__global__ __launch_bounds__(smx::opmod::kThreads) void symmetrix_m0_reverse_v1(SymmetrixJitM0ArgsV1 args) {
    smx::opmod::m0_reverse<kChannels, kInputs, Table>(args);
}
#else
__global__ __launch_bounds__(smx::opmod::kThreads) void symmetrix_r0_density_prepare_v1(SymmetrixJitR0ArgsV1 args) {
    smx::opmod::r0_density_prepare(args);
}
__global__ __launch_bounds__(smx::opmod::kThreads) void symmetrix_r0_forward_v1(SymmetrixJitR0ArgsV1 args) {
    smx::opmod::r0_forward<kChannels, SMX_OPMOD_LMAX>(args);
}
__global__ __launch_bounds__(smx::opmod::kThreads) void symmetrix_r0_reverse_prepare_v1(SymmetrixJitR0ArgsV1 args) {
    smx::opmod::r0_reverse_prepare<kChannels, SMX_OPMOD_LMAX>(args);
}
__global__ __launch_bounds__(smx::opmod::kThreads) void symmetrix_r0_coordinate_reverse_v1(
    SymmetrixJitR0ArgsV1 args) {
    smx::opmod::r0_coordinate_reverse<kChannels, SMX_OPMOD_LMAX>(args);
}
#endif
}  // extern "C"
