"""Matrix-Game-3.0 call surface (wan/modules/ in the reference)."""
