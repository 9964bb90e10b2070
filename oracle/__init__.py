"""CPU oracle (test infrastructure only; the product package never imports it)."""
