"""vectorstorekit_amd -- MI355X (gfx950) search hot path of VectorStoreKit.

Hand-written HIP kernels behind the C ABI of include/vsk_hip.h
(``lib/libvsk_hip.so``), with a Python mirror of the reference's
accelerator, index and quantizer interfaces on top.
"""
from ._lib import VSKError, library_path, load_library  # noqa: F401
from .engine import (  # noqa: F401
    Context,
    DistanceComputeBackend,
    DistanceMetric,
    HIPAccelerationConfiguration,
    HIPAccelerationEngine,
    HIPAcceleratorStrategy,
    QuantizationMetadata,
    QuantizationParameters,
    QuantizationScheme,
    QuantizedVector,
    VectorDatabase,
)
from .clustering import (  # noqa: F401,E402
    ClusteringResult,
    KMeansClustering,
    KMeansClusteringConfiguration,
)
from .ivf import IVFConfiguration, IVFIndex  # noqa: F401,E402
from .quantization import (  # noqa: F401,E402
    BinaryDatabase,
    BinaryQuantizer,
    ProductQuantizer,
    ScalarQuantizer,
    SQ8Database,
)
