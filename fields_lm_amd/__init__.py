"""fields_lm_amd — MI355X (gfx950) native Field-block hot path of Fields LM.

The package directory is the importable spelling of ``fields-lm_amd`` (a hyphen cannot appear
in a Python module name).

Public surface (mirrors src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py):

* ``fused_field_read(raw, transition_r, transition_i, gamma, block_c, chunk_t)``
* ``IndependentVacancyField``, ``FieldBlock``, ``RMSNorm``, ``PackedSwiGLU``
* ``field_scan`` (with state_in / state_out) and ``field_decode_step`` (decode token loop)
* ``field_scan_norm`` / ``field_decode_norm_step``: the same with the mixer's read_norm fused
"""
from .field import (  # noqa: F401
    ScanPlan,
    BACKENDS,
    VAC_MAX,
    FieldBlock,
    IndependentVacancyField,
    PackedSwiGLU,
    RMSNorm,
    boundary_scan,
    field_decode_norm_step,
    field_decode_step,
    field_scan,
    field_scan_backward,
    field_scan_norm,
    gate_residual_norm,
    swiglu,
    fused_field_read,
    state_to_complex,
)

from .model import (  # noqa: F401,E402
    OFFICIAL_ARCHITECTURE,
    FieldsConfig,
    FieldsForCausalLM,
    FieldsForwardOutput,
    FieldTokenSystem,
    build_official_fields,
)

__version__ = "0.1.0"
