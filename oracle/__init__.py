"""CPU oracle package (test infrastructure only; the product never imports it)."""
