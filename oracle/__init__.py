"""CPU oracle: test infrastructure only (never imported by product code)."""
