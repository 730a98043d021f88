"""vLLM adapter: decode query packing and Index-K ingestion on the device."""
