"""CPU oracle of the paged KV-cache path (test infrastructure: the checker, never the product)."""
