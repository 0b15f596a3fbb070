"""CPU oracle (test infrastructure only; see qwen35_oracle.py)."""
