"""Minimal engine for the end-to-end configuration: a random-initialised Llama
model over the paged HIP path, the reference's continuous-batching scheduler,
a runner with captured decode graphs, and a greedy generate loop."""
