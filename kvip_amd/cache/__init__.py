"""Device-resident cache state: ABC ring maps and the resident-slot LRU."""
