"""MI355X (gfx950) HIP implementation of mini-EP's GraniteMoE MoE-block hot path.

Host-side mirror of the reference's MoE-backend API (miniep/modeling.py,
miniep/ep.py, miniep/balancer.py) over the C ABI of ``include/miniep_amd.h``:

  route / HipMoEBackend / HipEPShareBackend / EmulatedEPMoEBackend / EPStats
  Placement (naive / from_plan / to_plan / experts_of_rank / reset_rr / dest_ranks)
  plan_balanced
  ExpertStore / apply_placement (expert weights in slots, live re-placement)
  ops: router_topk, topk_softmax, dispatch, grouped_swiglu, combine
"""
from . import _lib, ops
from .backend import (EmulatedEPExchangeBackend, EmulatedEPMoEBackend, EPStats, HipEPShareBackend,
                      HipMoEBackend, SendBatch, route)
from .balancer import plan_balanced
from .placement import Placement
from .store import ExpertStore, apply_placement

__all__ = [
    "EmulatedEPExchangeBackend", "SendBatch",
    "_lib", "ops", "route", "HipMoEBackend", "HipEPShareBackend", "EmulatedEPMoEBackend",
    "EPStats", "Placement", "plan_balanced", "ExpertStore", "apply_placement",
]
