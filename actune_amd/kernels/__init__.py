"""Group-64 grouped backend modules, weight codebooks and config selection."""
