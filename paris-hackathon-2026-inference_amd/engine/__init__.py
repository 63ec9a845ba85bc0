"""MI355X-native Gated DeltaNet path, laid out like the reference's ``engine``
package so that ``from engine.kernels import chunk_gated_delta_rule`` resolves
here when ``paris-hackathon-2026-inference_amd/`` is on ``sys.path``."""
