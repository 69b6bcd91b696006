"""Host bookkeeping around the compression step."""
