"""Engine host around the paged KV path: sequences, pages, scheduling, model runner."""
