"""CPU oracle for the prefill hot path: test infrastructure, never the product path."""
