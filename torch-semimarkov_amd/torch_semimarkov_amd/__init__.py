"""torch_semimarkov_amd -- the streaming semi-Markov CRF scan of torch-semimarkov,
built for AMD Instinct MI355X (gfx950) with hand-written HIP kernels.

Public API (same names and meanings as the reference package for this path):

* :func:`semi_crf_streaming_forward` -- log partition / Viterbi score with autograd
* :class:`SemiMarkovCRFHead` -- ``forward`` / ``compute_loss`` / ``decode`` /
  ``decode_with_traceback``
* :class:`Segment`, :class:`ViterbiResult`, :func:`score_gold_vectorized`
* :func:`compute_edge_block_streaming`, :class:`SemiCRFStreamingHIP`
* :class:`UncertaintyMixin`, :class:`UncertaintySemiMarkovCRFHead` -- boundary /
  position marginals, streaming entropy, uncertainty-weighted loss
* :func:`emission_cum_scores` -- projected scores to cumulative scores on the GPU
* :func:`semi_crf_emissions_forward`, :func:`score_gold_emissions` -- the scan and
  the gold-path score on projected scores, with the prefix sums fused into the
  kernels (what the head's ``compute_loss`` / ``decode`` run)
"""

from .duration import DurationDistribution, LearnedDuration
from .helpers import Segment, ViterbiResult, score_gold_emissions, score_gold_vectorized
from .nn import SemiMarkovCRFHead
from .streaming import (
    HAS_HIP,
    NEG_INF,
    SemiCRFStreamingHIP,
    compute_edge_block_streaming,
    emission_cum_scores,
    semi_crf_emissions_forward,
    semi_crf_streaming_forward,
)
from .uncertainty import UncertaintyMixin, UncertaintySemiMarkovCRFHead

__version__ = "0.1.0"

__all__ = [
    "semi_crf_streaming_forward",
    "SemiCRFStreamingHIP",
    "compute_edge_block_streaming",
    "SemiMarkovCRFHead",
    "Segment",
    "ViterbiResult",
    "score_gold_vectorized",
    "DurationDistribution",
    "LearnedDuration",
    "NEG_INF",
    "HAS_HIP",
    "UncertaintyMixin",
    "UncertaintySemiMarkovCRFHead",
    "emission_cum_scores",
    "semi_crf_emissions_forward",
    "score_gold_emissions",
]
