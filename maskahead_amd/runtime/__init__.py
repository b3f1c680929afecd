"""Session-level pieces of the read/keep path (the reference's maskahead.runtime)."""
