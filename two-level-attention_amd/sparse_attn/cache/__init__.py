from .paged_region_cache import (
    GraphReadyPagedRegionCache,
    GraphReadyPagedRegionLayer,
    RequestPhase,
    RequestState,
    SINK, FAR, NEAR, SWA,
)
