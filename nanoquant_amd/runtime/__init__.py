"""Runtime surface for the packed linear: backend contract, layout, backend
selection, module binding and the HIP backend (the contract and layout keep the
names of the reference's ``nanoquant.runtime`` for this path)."""

from nanoquant_amd.runtime.backend import (
    BackendCapabilities,
    PreparedLayer,
    ProjectionMemberSpec,
    QuantizedLinearSpec,
    RuntimeBackend,
    RuntimeLayerState,
    SupportResult,
    WorkloadSpec,
    evaluate_capabilities,
)
from nanoquant_amd.runtime.constants import RUNTIME_ARTIFACT_SCHEMA_VERSION, PackedLayout
from nanoquant_amd.runtime.hip_backend import (
    HIP_PACKED_BACKEND_NAME,
    HIP_PACKED_BACKEND_VERSION,
    HipPackedBackend,
    HipProjectionGroup,
    grouped_hip_projection,
    prepare_hip_projection_group,
    unpack_sign_matrix_device,
)
from nanoquant_amd.runtime.logical import (
    LogicalLayerState,
    canonical_torch_dtype,
    parse_torch_dtype,
)
from nanoquant_amd.runtime.packed import (
    GGUF_TENSOR_SUFFIXES,
    PACKED_LAYOUT_VERSION,
    PACKED_REFERENCE_COMMIT,
    PACKED_REFERENCE_CUDA_SHA256,
    PACKED_TENSOR_NAMESPACE,
    PACKED_WORD_BITS,
    PackedLayerState,
    PackedLayoutMetadata,
    PackedReferenceProvenance,
    pack_logical_layer,
    pack_sign_matrix,
    packed_row_stride_bytes,
    packed_word_count,
    supports_vector_word_loads,
    unpack_sign_matrix,
)
from nanoquant_amd.runtime.dispatch import (
    Choice,
    PreparedModel,
    Rejection,
    SelectionError,
    choose_backends,
)
from nanoquant_amd.runtime.decoder_shell import (
    DecodeStep,
    DecoderLayerWeights,
    DecoderShellConfig,
    DecoderShellError,
    DecoderShellWeights,
    PackedDecoder,
)
from nanoquant_amd.runtime.packed_artifact import (
    OpenPackedArtifact,
    PackedArtifactError,
    PackedModelManifest,
    RuntimeModelMetadata,
    open_packed_artifact,
    write_packed_artifact,
)
from nanoquant_amd.runtime.row_sidecar import OutputRowSidecar, RowSidecarLayerState
from nanoquant_amd.runtime.torch_model import (
    PreparedLinear,
    PreparedProjectionView,
    bind_prepared_linears,
    execution_workload,
    transformers_decoder_module_paths,
)

__all__ = [name for name in dir() if not name.startswith("_")]
