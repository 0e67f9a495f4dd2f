"""Test-only CPU oracle (see tq_oracle.py).  Never imported by the product path."""
