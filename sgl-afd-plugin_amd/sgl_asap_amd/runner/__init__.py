"""F-side job handling: scheduler run_job and HIP-graph buckets."""
