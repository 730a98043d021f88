"""LIFetch: lightning-indexer scoring -> TopK-2048 -> Fetch, one graph-capturable forward."""
