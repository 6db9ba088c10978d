"""vLLM-v1-shaped front end of the device sampler: metadata, sampler facade, runner, worker."""
