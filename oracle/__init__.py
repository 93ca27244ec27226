"""Test-only oracle for the paged KV-cache path (see oracle/paged_ref.py). Never imported by the product."""
