"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference training path (parity checker, never the product)."""
