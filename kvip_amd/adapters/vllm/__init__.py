"""vLLM adapter: decode query packing, Index-K ingestion and the indexer selector."""
