"""gru_qat_amd: MI355X-native persistent GRU scan (forward on hand-written
gfx950 HIP kernels behind the C ABI of libgruscan.so).

Drop-in replacements for the scan entry points of LarocheC/gru-triton
(gru_qat.triton_kernels.scan*), keeping their names, signatures and error
types.
"""

from .scan import (
    GRUScanFunction,
    GRUScanPersistentFunction,
    gru_scan,
    gru_scan_forward,
    gru_scan_forward_persistent,
    gru_scan_persistent,
)
from .scan_butterfly import (
    extract_butterfly_twiddles,
    gru_scan_butterfly_forward,
    gru_scan_butterfly_persistent,
    gru_scan_butterfly_triton,
)
from .scan_diagonal import extract_diagonal_factors, gru_scan_diagonal, gru_scan_diagonal_forward
from .scan_monarch import extract_monarch_factors, gru_scan_monarch, gru_scan_monarch_forward
from .scan_circulant import extract_circulant_factors, gru_scan_circulant, gru_scan_circulant_forward
from ._common import set_save_gh
from ._lib import PersistentScanFault, check_faults, load as load_library, workspace_faults
from .gru_layer import ScanLayer, fast_dispatch_eligible, forward_fast_dispatch, layer_forward, resolve_use_triton
from .input_proj import input_projection, quantize_input_weights
from .struct_proj import structured_input_projection
from .quantizers import FakeQuantizePerTensor, QuantizerConfig
from .observe import gru_scan_observe, hidden_map_dense
from .calibration import calibrate, freeze_all
from .export import dequantize_int_weights, export_int_weights, quantize_rows

__all__ = [
    "FakeQuantizePerTensor",
    "GRUScanFunction",
    "GRUScanPersistentFunction",
    "QuantizerConfig",
    "ScanLayer",
    "calibrate",
    "dequantize_int_weights",
    "export_int_weights",
    "extract_butterfly_twiddles",
    "extract_diagonal_factors",
    "extract_monarch_factors",
    "fast_dispatch_eligible",
    "freeze_all",
    "forward_fast_dispatch",
    "gru_scan",
    "gru_scan_butterfly_forward",
    "gru_scan_butterfly_persistent",
    "gru_scan_butterfly_triton",
    "gru_scan_diagonal",
    "gru_scan_diagonal_forward",
    "gru_scan_forward",
    "gru_scan_forward_persistent",
    "gru_scan_monarch",
    "gru_scan_monarch_forward",
    "gru_scan_observe",
    "gru_scan_persistent",
    "hidden_map_dense",
    "input_projection",
    "layer_forward",
    "load_library",
    "quantize_input_weights",
    "quantize_rows",
    "resolve_use_triton",
    "workspace_faults",
    "structured_input_projection",
    "gru_scan_circulant",
    "gru_scan_circulant_forward",
    "extract_circulant_factors",
    "check_faults",
    "PersistentScanFault",
    "set_save_gh",
]
