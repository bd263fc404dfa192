"""Test-side stand-in for the reference repository's ``benchmarks`` package (its harness).

Only ``benchmarks.workloads`` is provided, mapped onto the package's
``sglang_decode.workloads``, so tests written against the reference's imports run here.
"""
