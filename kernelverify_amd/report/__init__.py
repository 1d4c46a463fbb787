"""Verification certificates for the pack kernels (reference: kernelverify/report/)."""

from kernelverify_amd.report.certificate import (  # noqa: F401
    EXTRACTED_UNVALIDATED,
    EXTRACTED_VALIDATED,
    NUMERIC,
    OWN_SOURCE,
    SCHEMA_VERSION,
    STRUCTURAL,
    WRAPPER_ASSEMBLED,
    Certificate,
    ClauseAttestation,
    EmitReport,
    PerformanceClaim,
    audit,
    emit,
    render_markdown,
)
