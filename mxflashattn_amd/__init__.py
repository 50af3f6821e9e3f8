"""MI355X-native split-KV paged decode behind the MXFlashAttn API."""
