"""One speculative step of SimSD on one MI355X, built on the kernels of this
package: the draft's block denoising, the target's multi-block cached verify
with greedy acceptance, and the synthetic SDAR-shape models they run."""
