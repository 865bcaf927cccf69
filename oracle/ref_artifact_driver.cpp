// Command-line driver over the REFERENCE artifact code -- TEST INFRASTRUCTURE
// ONLY.  Linked with the reference's own src/artifact/{writer,reader,
// checksum,metadata}.cpp (compiled where they lie, see Makefile target `ref`)
// into oracle/_ref/artifact_ref, so the tests can compare this build's reader,
// writer and CRC-64 with the reference's on the same files.
//
//   artifact_ref write OUT META_JSON_FILE [NAME TYPE PAYLOAD_FILE]...
//       ArtifactWriter::set_raw_metadata_json + add_section + write_to_file
//   artifact_ref dump IN
//       ArtifactReader::open, validate_checksum, read_section of every
//       section; prints one JSON object (header, footer, sections, results)
//   artifact_ref crc FILE
//       Crc64 over the whole file (prints the value in hex)
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "artifact/checksum.h"
#include "artifact/reader.h"
#include "artifact/writer.h"

using namespace xinfer::artifact;

static std::vector<uint8_t> slurp(const char* path) {
    std::ifstream in(path, std::ios::binary);
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
}

static std::string json_str(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += (char)c;
        } else if (c < 0x20) {
            char b[8];
            std::snprintf(b, sizeof(b), "\\u%04x", c);
            o += b;
        } else {
            o += (char)c;
        }
    }
    return o + "\"";
}

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    const std::string cmd = argv[1];
    if (cmd == "write") {
        if (argc < 4 || (argc - 4) % 3 != 0) return 2;
        ArtifactWriter w;
        const std::vector<uint8_t> meta = slurp(argv[3]);
        w.set_raw_metadata_json(std::string(meta.begin(), meta.end()));
        for (int i = 4; i + 2 < argc; i += 3) {
            std::vector<uint8_t> payload = slurp(argv[i + 2]);
            if (!w.add_section(argv[i], static_cast<SectionType>(std::stoul(argv[i + 1])), std::move(payload))) {
                std::printf("{\"ok\": false, \"error\": \"add_section %s\"}\n", argv[i]);
                return 1;
            }
        }
        std::string err;
        const bool ok = w.write_to_file(argv[2], &err);
        std::printf("{\"ok\": %s, \"error\": %s}\n", ok ? "true" : "false", json_str(err).c_str());
        return ok ? 0 : 1;
    }
    if (cmd == "dump") {
        ArtifactReader r;
        std::string err;
        if (!r.open(argv[2], &err)) {
            std::printf("{\"open\": false, \"error\": %s}\n", json_str(err).c_str());
            return 0;
        }
        std::string verr;
        const bool valid = r.validate_checksum(&verr);
        const FileHeader& h = r.header();
        std::printf("{\"open\": true, \"valid\": %s, \"validate_error\": %s, ", valid ? "true" : "false",
                    json_str(verr).c_str());
        std::printf("\"header\": {\"format_version\": %u, \"section_count\": %u, \"metadata_offset\": %llu, "
                    "\"metadata_size\": %llu, \"section_table_offset\": %llu, \"total_file_size\": %llu}, ",
                    h.format_version, h.section_count, (unsigned long long)h.metadata_offset,
                    (unsigned long long)h.metadata_size, (unsigned long long)h.section_table_offset,
                    (unsigned long long)h.total_file_size);
        std::printf("\"footer_checksum\": \"%016llx\", \"metadata\": %s, \"sections\": [",
                    (unsigned long long)r.footer().file_checksum, json_str(r.raw_metadata_json()).c_str());
        bool first = true;
        for (const std::string& name : r.list_sections()) {
            const auto info = r.get_section_info(name);
            std::vector<uint8_t> data;
            std::string rerr;
            const bool rok = r.read_section(name, data, &rerr);
            std::printf("%s{\"name\": %s, \"type\": %u, \"flags\": %u, \"offset\": %llu, \"size\": %llu, "
                        "\"checksum\": \"%016llx\", \"read_ok\": %s, \"read_error\": %s}",
                        first ? "" : ", ", json_str(name).c_str(), info->type_tag, info->flags,
                        (unsigned long long)info->offset, (unsigned long long)info->size,
                        (unsigned long long)info->checksum, rok ? "true" : "false", json_str(rerr).c_str());
            first = false;
        }
        std::printf("]}\n");
        return 0;
    }
    if (cmd == "crc") {
        const std::vector<uint8_t> d = slurp(argv[2]);
        std::printf("%016llx\n", (unsigned long long)Crc64::calculate(d.data(), d.size()));
        return 0;
    }
    return 2;
}
