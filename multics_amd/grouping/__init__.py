"""Membership producer: player poses -> per-frame local groups (the
``membership`` / ``global_only`` topology the hierarchical mask builders take)
and the 24-field ``groups.pt`` label payload (multics/grouping/*).

CPU work, once per 165-frame clip: a few hundred [P, P] pose matrices and a
beam search over at most ten players per 48-frame period.

* ``state``      -- ``GroupingState`` (the ``grouping_state.npz`` format)
* ``budget``     -- communication budget / topology costs (``resolve``)
* ``relevance``  -- pose-only pair relevance per period
* ``partition``  -- bounded clique cover (``flexible_partition``)
* ``labels``     -- ``generate_labels``, ``track_labels``, ``membership_inputs``
* ``validation`` -- ``validate_generated_labels``, ``validate_existing_labels``
* ``files``      -- ``load_group_labels``, ``save_group_labels``
"""

from .budget import Budget, resolve
from .labels import generate_labels, membership_inputs, track_labels
from .partition import FlexGrouping, flexible_partition
from .relevance import history_components, relevance_periods
from .state import GroupingState, eligible_players
from .validation import validate_existing_labels, validate_generated_labels
from .files import load_group_labels, save_group_labels

__all__ = ["Budget", "resolve", "generate_labels", "membership_inputs", "track_labels",
           "FlexGrouping", "flexible_partition", "history_components", "relevance_periods",
           "GroupingState", "eligible_players", "validate_existing_labels",
           "validate_generated_labels", "load_group_labels", "save_group_labels"]
