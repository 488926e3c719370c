"""The KV handoff connector: wire codec, transports, RngdKVConnector."""
