"""HY-WorldPlay call surface (hyvideo/models/transformers/modules/ in the reference)."""
