"""CPU oracle for the pi0.5 denoise loop (test infrastructure; never imported by the product)."""
